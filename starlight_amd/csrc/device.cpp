// HipDevice: the MI355X implementation of StarLight's sl_device::Device
// contract (ARCH-0007 §3.1), exported through the C ABI in starlight_hip.h.
//
// It plays the role CpuDevice plays for backend-cpu
// (crates/backends/backend-cpu/src/device.rs:31-213):
//  * buffers are device allocations indexed by dense u32 ids, zero-filled at
//    allocation (device.rs:55-83);
//  * dispatch() validates exactly as CpuDevice does (validate.cpp) and logs
//    the accepted command; every error a reference dispatch reports is
//    reported here, at the same call;
//  * the log is submitted to the device's single stream before anything can
//    observe its effects: synchronize(), upload, download, bind_quantized
//    (and sl_hip_submit). Submission runs the commands in order, fusing
//    adjacent ones where one kernel can do their work (an RMSNorm into the
//    GEMVs that read its output, q/k/v GEMVs into one launch, a GEMV into
//    the residual Add after it, gate/up into one launch with the silu*up
//    epilogue); every command's outputs are still written. A log that
//    repeats the previous one (decode steps) is captured once as a HIP
//    graph and replayed; past_len reaches its kernels through a small device
//    array set before each submission, so one graph serves every step;
//  * synchronize() submits, then waits for the stream (CpuDevice's is a
//    no-op because it is synchronous); a kernel failure surfaces there.
// Ports that share a buffer (the sl-core scratchpad) are plain base + offset
// pointers; CpuDevice's take/restore staging (device.rs:379-706) has no GPU
// counterpart.
//
// U32 buffers are never written by a command (device.rs:311-316), only by
// upload_u32, so the device keeps a host copy of small ones and checks Gather
// ids before launching, like reference/layout.rs:207-213 checks them before
// its first write.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>
#include <utility>
#include <vector>

#include "kernels/kernels.h"
#include "internal.h"
#include "plan.h"
#include "starlight_hip.h"

namespace slhip {
namespace {

constexpr uint64_t kMirrorMaxElements = 1ull << 22;        // host copy of u32 buffers up to 16 MiB
constexpr uint64_t kSmallUploadWords = 64;                  // uploads carried in kernel arguments, at most
constexpr uint64_t kWorkspaceBytes = 512ull << 20;          // split-K partials, SwiGlu intermediates
constexpr uint64_t kRopeTableFloats = 16 * 512;  // tokens x head_dim of one decode submission
constexpr uint64_t kIdScratchElements = 1ull << 20;         // host scratch for unmirrored id checks

struct Buffer {
    sl_buffer_desc desc{};
    void* base = nullptr;  // allocation start
    void* ptr = nullptr;   // aligned data start
    std::vector<uint32_t> mirror;
    bool mirrored = false;
    // group-quantized binding
    uint32_t scales = 0;
    uint8_t* tiles = nullptr;  // private codes, then (Mfma) tile-ordered scales
    float* tile_scales = nullptr;
    QuantLayout layout = QuantLayout::RowMajor;
};

constexpr size_t kLogFlushLength = 8192;  // submit early past this many logged commands
constexpr size_t kGraphCacheSize = 16;

// An accepted command waiting for submission.
struct Logged {
    Plan plan;
    sl_buffer_ref in[kMaxInputs];
    sl_buffer_ref out;
    uint32_t n_in = 0;
    int32_t dyn_slot = -1;  // index of its past_len in the device array, if it reads one
};

struct GraphEntry {
    std::vector<uint64_t> key;
    uint64_t hash = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t last_use = 0;
};

}  // namespace

struct Device : BufferView {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    std::vector<Buffer> buffers;
    float* workspace = nullptr;
    uint64_t workspace_floats = 0;
    float* static_scratch = nullptr;  // this GPU's static array (no-allocation entry point)
    std::vector<uint32_t> id_scratch;
    Error last;
    // deferred submission
    std::vector<Logged> log;
    uint32_t options = SL_HIP_OPT_FUSION | SL_HIP_OPT_GRAPHS;
    uint32_t* dyn = nullptr;  // device past_len slots, kLogFlushLength of them
    std::vector<uint32_t> dyn_values;
    std::vector<uint32_t> paged_readers;  // host scratch of the paged-attention page check
    // State buffers bound to a paged cache (sl_hip_bind_paged_state)
    std::vector<std::pair<uint32_t, sl_paged_kv>> paged_states;
    const sl_paged_kv* paged_of(uint32_t state) const {
        for (const auto& p : paged_states)
            if (p.first == state) return &p.second;
        return nullptr;
    }
    std::vector<uint64_t> key, prev_key;
    std::vector<GraphEntry> graphs;
    size_t last_graph = SIZE_MAX;  // entry of graphs the previous replay or capture used
    uint64_t use_clock = 0;
    sl_hip_stats stats{};
    // Rope sine / cosine table shared by the fused attention units of a
    // submission (one per step: every layer rotates at the same positions)
    float* rope_tab = nullptr;
    struct {
        bool valid = false;
        sl_buffer_ref pos{};
        float theta = 0.f;
        uint64_t head_dim = 0, tokens = 0;
        size_t at = 0;  // log index where it was computed
    } rope;

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

sl_status flush(Device* d);

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
    if (d->buffers[id].desc.elements == len && len != 0 && flush(d) != SL_OK) return d->last.status;
    Buffer& b = d->buffers[id];
    if (b.desc.elements != len) return d->fail(Error::invalid_range(id, 0, len));
    if (len == 0) return SL_OK;
    bool feeds_copies = b.tiles != nullptr;
    if (kind == SL_BUFFER_F32)
        for (const Buffer& p : d->buffers) feeds_copies |= p.tile_scales != nullptr && p.scales == id;
    hipError_t e = hipSuccess;
    if (len <= kSmallUploadWords && !feeds_copies) {
        // A few words (token ids, positions of a decode step): written by a
        // kernel that carries them in its arguments, in stream order, so the
        // host neither stages a copy nor waits for it.
        e = launch_set_words(static_cast<uint32_t*>(b.ptr), static_cast<const uint32_t*>(data), len, d->stream);
    } else {
        e = hipMemcpyAsync(b.ptr, data, len * 4, hipMemcpyHostToDevice, d->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    }
    if (e != hipSuccess) return d->hip_fail(e);
    if (b.mirrored) std::memcpy(b.mirror.data(), data, len * 4);
    if (b.tiles) {
        // A re-uploaded quantized payload refreshes the private tile copy.
        e = launch_quant_repack(static_cast<const uint8_t*>(b.ptr), b.tiles, b.desc.qformat, b.desc.qn, b.desc.qk,
                                b.layout, d->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
        if (e != hipSuccess) return d->hip_fail(e);
    }
    if (kind == SL_BUFFER_F32) {
        // ... and re-uploaded scales refresh every tile-ordered copy made from them.
        for (const Buffer& p : d->buffers) {
            if (p.tile_scales == nullptr || p.scales != id) continue;
            e = launch_scale_repack(static_cast<const float*>(b.ptr), p.tile_scales, p.desc.qn, p.desc.qk,
                                    p.desc.group_size, d->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
            if (e != hipSuccess) return d->hip_fail(e);
        }
    }
    return SL_OK;
}

sl_status copy_out(Device* d, uint32_t id, void* out, size_t len, uint32_t kind) {
    if (id >= d->buffers.size() || d->buffers[id].desc.kind != kind) return d->fail(Error::invalid_buffer(id));
    if (d->buffers[id].desc.elements == len && len != 0 && flush(d) != SL_OK) return d->last.status;
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
    w.quant.tile_scales = b.tile_scales;
    w.quant.format = q.format;
    w.quant.group = q.group;
    w.quant.n = q.n;
    w.quant.k = q.k;
    return w;
}

// Enqueues the kernels of one validated command with `ws` as their scratch
// memory; `dyn`, when set, is the device word its kernels read past_len from.
hipError_t launch(Device* d, const Plan& p, const sl_buffer_ref* in, const sl_buffer_ref* out,
                  const uint32_t* dyn, const Workspace& ws) {
    hipStream_t s = d->stream;
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
            return launch_softmax(fptr(d, in[0]), fptr(d, out[0]), p.rows, p.cols, false, 0, 0, nullptr, s);
        case SL_OP_SOFTMAX_CAUSAL:
            return launch_softmax(fptr(d, in[0]), fptr(d, out[0]), p.rows, p.cols, true, p.seq, p.past_len, dyn, s);
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
                                    p.layer, p.kv_heads, p.head_dim, p.max_seq, p.past_len, p.seq, dyn, s);
        case SL_OP_CAUSAL_ATTENTION: {
            if (const sl_paged_kv* kv = d->paged_of(in[p.state_index].buffer)) {
                PagedAttentionArgs a{};
                a.q = fptr(d, in[0]);
                a.k_new = fptr(d, in[1]);
                a.v_new = fptr(d, in[2]);
                a.pool = static_cast<float*>(d->buffers[kv->pool].ptr);
                a.out = fptr(d, out[0]);
                a.block_table = static_cast<const uint32_t*>(d->buffers[kv->block_table].ptr);
                a.seq_lens = static_cast<const uint32_t*>(d->buffers[kv->seq_lens].ptr);
                a.batch = p.batch;
                a.layers = kv->layers;
                a.layer = p.layer;
                a.heads = p.heads;
                a.kv_heads = p.kv_heads;
                a.head_dim = p.head_dim;
                a.num_pages = kv->num_pages;
                a.page_size = kv->page_size;
                a.pages_per_seq = kv->pages_per_seq;
                a.scale = p.scale;
                if (paged_attention_workspace_floats(a) > ws.floats) return hipErrorNotSupported;
                return launch_paged_attention(a, ws, s);
            }
            AttentionArgs a{fptr(d, in[0]), fptr(d, in[1]), fptr(d, in[2]), fptr(d, in[p.state_index]),
                            fptr(d, out[0]), p.batch, p.layers, p.layer, p.heads, p.kv_heads, p.seq,
                            p.past_len, p.head_dim, p.max_seq, p.scale, dyn};
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

// Limits of the launch paths that validation does not know about, for a
// scratch area of `ws_floats`; checked before anything is enqueued so a
// rejected call still changes nothing.
bool device_limits(const Plan& p, uint64_t ws_floats, Error* err) {
    if (p.code == SL_OP_CAUSAL_ATTENTION && p.head_dim > 256) {
        *err = Error::unimplemented("head_dim above 256 is not supported by HipDevice");
        return false;
    }
    if (p.code == SL_OP_SWIGLU && 2 * p.inter > ws_floats / 2) {
        *err = Error::unimplemented("swiglu inter size exceeds the device workspace");
        return false;
    }
    if (p.code == SL_OP_RMS_NORM_MATMUL && p.hidden > ws_floats / 2) {
        *err = Error::unimplemented("rms_norm_matmul hidden size exceeds the device workspace");
        return false;
    }
    return true;
}

// ---- deferred submission: fusion, past_len slots, graph replay ----

bool reads_past(uint32_t code) {
    return code == SL_OP_SOFTMAX_CAUSAL || code == SL_OP_KV_APPEND || code == SL_OP_CAUSAL_ATTENTION;
}

bool overlaps(const sl_buffer_ref& a, const sl_buffer_ref& b) {
    return a.buffer == b.buffer && a.len != 0 && b.len != 0 && a.offset < b.offset + b.len &&
           b.offset < a.offset + a.len;
}
bool same_ref(const sl_buffer_ref& a, const sl_buffer_ref& b) {
    return a.buffer == b.buffer && a.offset == b.offset && a.len == b.len;
}

// Port `port` of `c` is a quantized weight in the MFMA tile layout.
bool mfma_weight(const Device* d, const Logged& c, size_t port) {
    if (!c.plan.quant[port].present) return false;
    const Buffer& b = d->buffers[c.in[port].buffer];
    return b.layout == QuantLayout::Mfma && b.tile_scales != nullptr;
}

// The paged cache's buffers: pool f32 of layers * num_pages * 2 * page_size
// * kv_heads * head_dim elements, block table and lengths u32 buffers with
// host copies, page_size a multiple of the decode tile.
bool check_paged_buffers(const Device* d, const sl_paged_kv& kv, uint64_t kv_heads, uint64_t head_dim,
                         Error* err) {
    if (kv.page_size == 0 || kv.page_size % 16 != 0) {
        *err = Error::unimplemented("page_size must be a nonzero multiple of 16");
        return false;
    }
    if (kv.layers == 0 || kv.num_pages == 0 || kv.pages_per_seq == 0) {
        *err = Error::execution("the page pool is empty");
        return false;
    }
    if (kv.pool >= d->buffers.size() || d->buffers[kv.pool].desc.kind != SL_BUFFER_F32) {
        *err = Error::invalid_buffer(kv.pool);
        return false;
    }
    for (uint32_t id : {kv.block_table, kv.seq_lens})
        if (id >= d->buffers.size() || d->buffers[id].desc.kind != SL_BUFFER_U32) {
            *err = Error::invalid_buffer(id);
            return false;
        }
    if (!d->buffers[kv.block_table].mirrored || !d->buffers[kv.seq_lens].mirrored) {
        *err = Error::unimplemented("block table and lengths must be u32 buffers of at most 16 MiB");
        return false;
    }
    if (kv_heads != 0 && d->buffers[kv.pool].desc.elements !=
                             static_cast<uint64_t>(kv.layers) * kv.num_pages * 2 * kv.page_size * kv_heads * head_dim) {
        *err = Error::execution("page pool size does not match its layout");
        return false;
    }
    return true;
}

// The block tables and lengths of rows 0..B-1, from the host copies: every
// position 0..L of a row maps to a page below num_pages, and the page a row
// appends into is read by no other row (rows run in parallel; pages shared
// read-only, such as a common prefix, are fine).
bool check_paged_tables(Device* d, const sl_paged_kv& kv, uint64_t B, Error* err) {
    const Buffer& tb = d->buffers[kv.block_table];
    const Buffer& lb = d->buffers[kv.seq_lens];
    if (tb.desc.elements < B * kv.pages_per_seq || lb.desc.elements < B) {
        *err = Error::execution("block table or lengths buffer is too small for the batch");
        return false;
    }
    for (uint64_t b = 0; b < B; ++b) {
        const uint64_t L = lb.mirror[b];
        if (L / kv.page_size >= kv.pages_per_seq) {
            *err = Error::execution("paged KV length exceeds the row's block table");
            return false;
        }
        for (uint64_t pi = 0; pi <= L / kv.page_size; ++pi)
            if (tb.mirror[b * kv.pages_per_seq + pi] >= kv.num_pages) {
                *err = Error::execution("page id out of range");
                return false;
            }
    }
    // readers[p]: the one row reading page p, kNone, or kShared for several
    constexpr uint32_t kNone = 0xffffffffu, kShared = 0xfffffffeu;
    std::vector<uint32_t>& readers = d->paged_readers;
    readers.assign(kv.num_pages, kNone);
    for (uint64_t b = 0; b < B; ++b)
        for (uint64_t pi = 0; pi <= lb.mirror[b] / kv.page_size; ++pi) {
            uint32_t& r = readers[tb.mirror[b * kv.pages_per_seq + pi]];
            r = (r == kNone || r == b) ? static_cast<uint32_t>(b) : kShared;
        }
    for (uint64_t b = 0; b < B; ++b)
        if (readers[tb.mirror[b * kv.pages_per_seq + lb.mirror[b] / kv.page_size]] != b) {
            *err = Error::execution("a row appends into a page another row reads");
            return false;
        }
    return true;
}

// A command on a State buffer bound to a paged cache: CausalAttention with
// one new token per row over pages that its shapes match.
bool check_paged_command(Device* d, const Plan& p, const sl_paged_kv& kv, Error* err) {
    if (p.code != SL_OP_CAUSAL_ATTENTION) {
        *err = Error::unimplemented("only CausalAttention reads a paged State on HipDevice");
        return false;
    }
    if (p.seq != 1) {
        *err = Error::unimplemented("a paged State takes one new token per row");
        return false;
    }
    if (p.head_dim == 0 || p.head_dim % 64 != 0 || p.head_dim > 256) {
        *err = Error::unimplemented("paged attention needs head_dim a multiple of 64 up to 256");
        return false;
    }
    if (p.heads / p.kv_heads > 16) {
        *err = Error::unimplemented("paged attention takes at most 16 query heads per KV head");
        return false;
    }
    if (p.layers != kv.layers) {
        *err = Error::execution("paged State layers do not match the page pool");
        return false;
    }
    return check_paged_buffers(d, kv, p.kv_heads, p.head_dim, err) && check_paged_tables(d, kv, p.batch, err);
}

// The paged decode arguments of a CausalAttention on a bound State.
void set_paged(const Device* d, const sl_paged_kv& kv, AttentionArgs* a) {
    a->cache = static_cast<float*>(d->buffers[kv.pool].ptr);
    a->block_table = static_cast<const uint32_t*>(d->buffers[kv.block_table].ptr);
    a->seq_lens = static_cast<const uint32_t*>(d->buffers[kv.seq_lens].ptr);
    a->num_pages = kv.num_pages;
    a->page_size = kv.page_size;
    a->pages_per_seq = kv.pages_per_seq;
    a->max_seq = static_cast<uint64_t>(kv.pages_per_seq) * kv.page_size;
    a->past_len = 0;
    a->dyn = nullptr;
}

// An Add right after a command that wrote `o` (rows * n values), adding it to
// another operand: returns the port of that other operand, or -1. The Add's
// output overlaps neither of its inputs (dispatch validation rejects that)
// and must not overlap the inputs the fused kernel still reads. The residual
// operand is read early by every block, so it must not overlap `o` or
// `written`, a region the fused kernel writes before its epilogue (the norm
// output block 0 writes in its prologue).
int residual_port(const Logged& a, const sl_buffer_ref& o, uint64_t count, const sl_buffer_ref* reads,
                  size_t n_reads, const sl_buffer_ref* written = nullptr) {
    if (a.plan.code != SL_OP_ADD || a.plan.len != count) return -1;
    int other = same_ref(a.in[1], o) ? 0 : same_ref(a.in[0], o) ? 1 : -1;
    if (other < 0 || overlaps(a.in[other], o) || overlaps(a.out, o) || overlaps(a.out, a.in[other])) return -1;
    if (written != nullptr && overlaps(a.in[other], *written)) return -1;
    for (size_t i = 0; i < n_reads; ++i)
        if (overlaps(a.out, reads[i])) return -1;
    return other;
}

// Whether `r` is dead after log[from..] (defined with the attention fusion below).
bool dead_after(const Device* d, size_t from, const sl_buffer_ref& r, size_t skip_reads = SIZE_MAX);

// Tries to run log[i..] as one fused unit; returns the number of commands it
// covered (0: nothing launched, run log[i] alone).
size_t try_fuse(Device* d, size_t i, hipError_t* err) {
    const size_t n = d->log.size();
    const Logged* norm = nullptr;
    size_t j = i;
    if (d->log[i].plan.code == SL_OP_RMS_NORM) {
        norm = &d->log[i];
        j = i + 1;
        if (j >= n || overlaps(norm->out, norm->in[0]) || overlaps(norm->out, norm->in[1])) return 0;
    }
    const Logged& c1 = d->log[j];
    if (norm && !same_ref(c1.in[0], norm->out)) return 0;
    const sl_buffer_ref a_ref = norm ? norm->in[0] : c1.in[0];  // what the fused kernel reads
    sl_buffer_ref reads[3] = {a_ref, norm ? norm->in[1] : a_ref, norm ? norm->out : a_ref};
    const size_t n_reads = 3;
    QgemvFused f{};
    f.a = fptr(d, a_ref);
    f.partial = d->workspace;  // the unit uses no other workspace
    f.partial_floats = d->workspace_floats;
    if (norm) {
        f.gamma = fptr(d, norm->in[1]);
        f.normed = fptr(d, norm->out);
        f.eps = norm->plan.eps;
    }
    QuantWeight w[kFusedMaxSegs];

    if (c1.plan.code == SL_OP_MATMUL_NT && mfma_weight(d, c1, 1)) {
        const uint64_t rows = c1.plan.batch * c1.plan.m, k = c1.plan.k;
        if (rows == 0 || (norm && (norm->plan.rows != rows || norm->plan.hidden != k))) return 0;
        sl_buffer_ref outs[kFusedMaxSegs];
        uint32_t cnt = 0;
        for (size_t t = j; t < n && cnt < kFusedMaxSegs; ++t) {
            const Logged& c = d->log[t];
            if (c.plan.code != SL_OP_MATMUL_NT || !mfma_weight(d, c, 1) || !same_ref(c.in[0], c1.in[0]) ||
                c.plan.batch * c.plan.m != rows || c.plan.k != k)
                break;
            bool clash = false;
            for (size_t r = 0; r < n_reads; ++r) clash = clash || overlaps(c.out, reads[r]);
            for (uint32_t u = 0; u < cnt; ++u) clash = clash || overlaps(c.out, outs[u]);
            if (clash) break;
            w[cnt] = weight_ref(d, c.in[1], c.plan.quant[1]).quant;
            outs[cnt] = c.out;
            f.w[cnt] = &w[cnt];
            f.out[cnt] = fptr(d, c.out);
            ++cnt;
        }
        if (cnt == 0) return 0;
        size_t used = (j - i) + cnt;
        f.nseg = cnt;
        f.m = rows;
        f.epilogue = kFusedPlain;
        const Logged* add = cnt == 1 && j + 1 < n ? &d->log[j + 1] : nullptr;
        const uint64_t count = rows * w[0].n;
        auto set_residual = [&](int other) {
            f.epilogue = other >= 0 ? kFusedResidual : kFusedPlain;
            if (other >= 0) {
                f.resid[0] = fptr(d, add->in[other]);
                f.out2[0] = fptr(d, add->out);
            }
        };
        // Few rows: one fused GEMV launch, whose blocks read the activations
        // (and block 0 writes the norm output) while others write results.
        const int other = add ? residual_port(*add, outs[0], count, reads, n_reads, norm ? &norm->out : nullptr) : -1;
        hipError_t e = hipErrorNotSupported;
        if (used + (other >= 0 ? 1 : 0) > 1) {
            set_residual(other);
            e = launch_qgemv_fused(f, d->stream);
        }
        if (e != hipErrorNotSupported) {
            if (other >= 0) ++used;
            *err = e;
            d->stats.fused_commands += used;
            return used;
        }
        // Many rows (prefill): the projections as one q-GEMM launch over one
        // activation split for all of them, a residual Add in its epilogue.
        // The norm runs inside the split when nothing after the unit reads
        // its output, else on its own first. The split copies the
        // activations into the workspace before the GEMM starts, so the
        // Add's output may reuse their space.
        if (rows <= 16) return 0;  // few rows the fused GEMV did not take: one launch each
        const int other_many = add ? residual_port(*add, outs[0], count, nullptr, 0) : -1;
        if (used + (other_many >= 0 ? 1 : 0) == 1) return 0;
        const Workspace ws{d->workspace, d->workspace_floats};
        const float* a = norm ? fptr(d, norm->out) : f.a;
        if (!qgemm_mfma_takes(a, f.w, cnt, rows, ws)) return 0;
        set_residual(other_many);
        const bool residual = other_many >= 0;
        if (residual) ++used;
        // the product itself, when nothing after the Add reads it, is not written
        if (residual && dead_after(d, i + used, outs[0])) f.out[0] = nullptr;
        // (dead from the command after its last reader on: the unit's Add,
        // which may overwrite it, counts)
        const bool norm_in_split = norm && qgemm_norm_takes(k, f.gamma) && qgemm_mfma_takes(f.a, f.w, cnt, rows, ws) &&
                                   dead_after(d, j + cnt, norm->out);
        e = norm && !norm_in_split ? launch_rms_norm(f.a, f.gamma, f.normed, rows, k, f.eps, d->stream) : hipSuccess;
        if (e == hipSuccess)
            e = launch_qgemm_multi(norm_in_split ? f.a : a, f.w, f.out, cnt, rows, ws, d->stream, nullptr,
                                   residual ? f.resid : nullptr, residual ? f.out2 : nullptr,
                                   norm_in_split ? f.gamma : nullptr, f.eps);
        *err = e;
        d->stats.fused_commands += used;
        return used;
    }

    if (c1.plan.code == SL_OP_SWIGLU && mfma_weight(d, c1, 1) && mfma_weight(d, c1, 2) &&
        c1.plan.quant[3].present) {
        const uint64_t rows = c1.plan.rows, hidden = c1.plan.hidden, inter = c1.plan.inter;
        if (rows == 0 || rows * inter > d->workspace_floats / 2 ||
            (norm && (norm->plan.rows != rows || norm->plan.hidden != hidden)))
            return 0;
        for (size_t r = 0; r < n_reads; ++r)
            if (overlaps(c1.out, reads[r])) return 0;
        // gate/up pair into the workspace (h = silu(g) * u) ...
        float* h = d->workspace;
        w[0] = weight_ref(d, c1.in[1], c1.plan.quant[1]).quant;
        w[1] = weight_ref(d, c1.in[2], c1.plan.quant[2]).quant;
        f.w[0] = &w[0];
        f.w[1] = &w[1];
        f.out[0] = h;
        f.nseg = 2;
        f.m = rows;
        f.epilogue = kFusedPair;
        hipError_t e = launch_qgemv_fused(f, d->stream);
        if (e == hipErrorNotSupported) {
            if (rows <= 16) return 0;
            // Many rows (prefill): the norm on its own, then the SwiGlu
            // composite (gate and up as one q-GEMM, silu(g) * u formed by
            // the down projection's activation split) with the residual Add
            // in the down projection's epilogue when one follows.
            // Each row chunk's activations are split into the workspace
            // before its products run, so the Add's output may reuse their
            // space, unless it is shifted against them and a later chunk
            // still reads rows an earlier chunk's Add wrote.
            // The norm runs inside the gate/up split when nothing after the
            // unit reads its output and every row chunk takes that route
            // (launch_swiglu then launches nothing else first), else on its own.
            size_t used = (j - i) + 1;
            const Logged* add = j + 1 < n ? &d->log[j + 1] : nullptr;
            const sl_buffer_ref x_ref = norm ? norm->out : c1.in[0];
            int other = add ? residual_port(*add, c1.out, rows * hidden, nullptr, 0) : -1;
            if (other >= 0 && overlaps(add->out, x_ref) && !same_ref(add->out, x_ref) &&
                swiglu_chunk_rows(d->workspace_floats, inter) < rows)
                other = -1;
            // with the norm in the split, the chunks read its input instead
            // (its output is dead from the command after the SwiGlu on: the
            // unit's Add, which may overwrite it, counts)
            const bool fold = norm && !(other >= 0 && overlaps(add->out, norm->in[0]) &&
                                        !same_ref(add->out, norm->in[0]) &&
                                        swiglu_chunk_rows(d->workspace_floats, inter) < rows) &&
                              dead_after(d, j + 1, norm->out);
            const auto run = [&](bool in_split) {
                return launch_swiglu(in_split ? f.a : norm ? f.normed : f.a, weight_ref(d, c1.in[1], c1.plan.quant[1]),
                                     weight_ref(d, c1.in[2], c1.plan.quant[2]),
                                     weight_ref(d, c1.in[3], c1.plan.quant[3]), fptr(d, c1.out), rows, hidden, inter,
                                     Workspace{d->workspace, d->workspace_floats}, d->stream,
                                     other >= 0 ? fptr(d, add->in[other]) : nullptr,
                                     other >= 0 ? fptr(d, add->out) : nullptr,
                                     other >= 0 && dead_after(d, i + used + 1, c1.out), in_split ? f.gamma : nullptr,
                                     f.eps);
            };
            e = fold ? run(true) : hipErrorNotSupported;
            if (e == hipErrorNotSupported) {
                e = norm ? launch_rms_norm(f.a, f.gamma, f.normed, rows, hidden, f.eps, d->stream) : hipSuccess;
                if (e == hipSuccess) e = run(false);
            }
            if (other >= 0) ++used;
            *err = e;
            d->stats.fused_commands += used;
            return used;
        }
        if (e != hipSuccess) {
            *err = e;
            return 1;
        }
        size_t used = (j - i) + 1;
        // ... then the down projection, with the residual Add when one follows
        const WeightRef down = weight_ref(d, c1.in[3], c1.plan.quant[3]);
        QgemvFused g{};
        g.a = h;
        w[2] = down.quant;
        g.w[0] = &w[2];
        g.out[0] = fptr(d, c1.out);
        g.nseg = 1;
        g.m = rows;
        g.epilogue = kFusedPlain;
        g.partial = d->workspace + d->workspace_floats / 2;  // past h
        g.partial_floats = d->workspace_floats / 2;
        // The down kernel reads only h (the workspace), the weights and, per
        // element, the residual: nothing another block could overwrite.
        if (j + 1 < n) {
            const Logged& a = d->log[j + 1];
            const int other = residual_port(a, c1.out, rows * hidden, nullptr, 0);
            if (other >= 0) {
                g.epilogue = kFusedResidual;
                g.resid[0] = fptr(d, a.in[other]);
                g.out2[0] = fptr(d, a.out);
            }
        }
        e = mfma_weight(d, c1, 3) ? launch_qgemv_fused(g, d->stream) : hipErrorNotSupported;
        if (e == hipErrorNotSupported) {
            const Workspace rest = Workspace{d->workspace, d->workspace_floats}.after(
                d->workspace_floats / 2);
            e = launch_linear(h, down, g.out[0], rows, hidden, inter, rest, d->stream);
        } else if (g.epilogue == kFusedResidual) {
            ++used;
        }
        *err = e;
        d->stats.fused_commands += used;
        return used;
    }
    return 0;
}

const uint32_t* dyn_of(const Device* d, const Logged& c) {
    return c.dyn_slot >= 0 ? d->dyn + c.dyn_slot : nullptr;
}

// True when every element of `r` is overwritten by commands log[from..]
// before any of them reads it: the value is dead, and a fused unit may skip
// writing it (the final contents are those later writes either way).
// `skip_reads` names a command whose reads do not count (one a fused unit
// redirects elsewhere).
bool dead_after(const Device* d, size_t from, const sl_buffer_ref& r, size_t skip_reads) {
    std::vector<std::pair<uint64_t, uint64_t>> live;
    if (r.len) live.push_back({r.offset, r.offset + r.len});
    for (size_t j = from; j < d->log.size() && !live.empty(); ++j) {
        const Logged& c = d->log[j];
        for (uint32_t k = 0; k < (j == skip_reads ? 0u : c.n_in); ++k) {
            const sl_buffer_ref& x = c.in[k];
            if (x.buffer != r.buffer || x.len == 0) continue;
            for (const auto& iv : live)
                if (x.offset < iv.second && iv.first < x.offset + x.len) return false;
        }
        const sl_buffer_ref& o = c.out;
        if (o.buffer != r.buffer || o.len == 0) continue;
        std::vector<std::pair<uint64_t, uint64_t>> rest;
        for (const auto& iv : live) {
            if (o.offset > iv.first) rest.push_back({iv.first, o.offset < iv.second ? o.offset : iv.second});
            if (o.offset + o.len < iv.second)
                rest.push_back({o.offset + o.len > iv.first ? o.offset + o.len : iv.first, iv.second});
        }
        live.clear();
        for (const auto& iv : rest)
            if (iv.first < iv.second) live.push_back(iv);
    }
    return live.empty();
}

// SplitHeads q/k/v, Rope q/k and CausalAttention (and MergeHeads, and the
// output projection with its residual Add) as the decode kernels with Rope
// applied inside: the split and rotated heads are never materialised, so
// the unit is taken only when each of them is dead (dead_after); the
// attention output and MergeHeads result are written unless dead. The
// projection reads a copy of the merged heads in the workspace, so its
// outputs may reuse any scratch region. Returns the commands covered.
size_t try_fuse_attention(Device* d, size_t i, hipError_t* err) {
    const size_t n = d->log.size();
    if (i + 6 > n) return 0;
    const Logged* c = &d->log[i];
    const Logged &sq = c[0], &sk = c[1], &sv = c[2], &rq = c[3], &rk = c[4], &at = c[5];
    if (sq.plan.code != SL_OP_SPLIT_HEADS || sk.plan.code != SL_OP_SPLIT_HEADS || sv.plan.code != SL_OP_SPLIT_HEADS ||
        rq.plan.code != SL_OP_ROPE || rk.plan.code != SL_OP_ROPE || at.plan.code != SL_OP_CAUSAL_ATTENTION)
        return 0;
    const Plan& ap = at.plan;
    const uint64_t B = ap.batch, S = ap.seq, H = ap.heads, Hkv = ap.kv_heads, D = ap.head_dim;
    auto split_ok = [&](const Logged& x, uint64_t heads) {
        return x.plan.batch == B && x.plan.seq == S && x.plan.heads == heads && x.plan.head_dim == D;
    };
    auto rope_ok = [&](const Logged& x, uint64_t heads) {
        return x.plan.batch == B && x.plan.seq == S && x.plan.heads == heads && x.plan.head_dim == D &&
               same_ref(x.in[1], rq.in[1]) && x.plan.theta == rq.plan.theta &&
               x.plan.rope_variant == rq.plan.rope_variant;
    };
    if (!split_ok(sq, H) || !split_ok(sk, Hkv) || !split_ok(sv, Hkv) || !rope_ok(rq, H) || !rope_ok(rk, Hkv) ||
        !same_ref(rq.in[0], sq.out) || !same_ref(rk.in[0], sk.out) || !same_ref(at.in[0], rq.out) ||
        !same_ref(at.in[1], rk.out) || !same_ref(at.in[2], sv.out))
        return 0;
    size_t used = 6;
    const Logged* mh = nullptr;
    if (i + 6 < n && c[6].plan.code == SL_OP_MERGE_HEADS && same_ref(c[6].in[0], at.out) &&
        c[6].plan.heads == H && c[6].plan.head_dim == D) {
        mh = &c[6];
        used = 7;
    }
    // The split and rotated heads are written only when a later command reads
    // them: each is scanned from the command after its last reader inside the
    // unit, so the unit's own later writes (the attention output, MergeHeads)
    // count as overwrites. The decode kernel writes a live one, so it must
    // not overlap anything that kernel reads or another live one; the
    // attention output and MergeHeads come from the merge kernel after it,
    // which keeps the op order where they overlap.
    // A live one that overlaps what the decode kernel reads, or another one
    // it writes, is staged instead: the kernel writes it to the workspace,
    // and once the unit's kernels are done its ranges that no later command
    // of the unit writes are copied to their place (the rotated q of a last
    // layer, whose tail nothing overwrites before the submission ends).
    const sl_buffer_ref& cache = at.in[ap.state_index];
    // what the kernels read and write of the cache: the State, or the page
    // pool bound to it
    const sl_paged_kv* paged = d->paged_of(cache.buffer);
    const sl_buffer_ref cache_ref =
        paged ? sl_buffer_ref{paged->pool, 0, 0, d->buffers[paged->pool].desc.elements} : cache;
    const sl_buffer_ref inter[5] = {sq.out, sk.out, sv.out, rq.out, rk.out};
    const size_t after_reader[5] = {i + 4, i + 5, i + 6, i + 6, i + 6};
    bool live[5], staged[5] = {false, false, false, false, false};
    for (int x = 0; x < 5; ++x) {
        live[x] = !dead_after(d, after_reader[x], inter[x]);
        if (!live[x]) continue;
        if (overlaps(inter[x], cache_ref)) return 0;
        const sl_buffer_ref read[4] = {sq.in[0], sk.in[0], sv.in[0], rq.in[1]};
        for (const sl_buffer_ref& t : read)
            if (overlaps(inter[x], t)) staged[x] = true;
        for (int y = 0; y < x; ++y)
            if (live[y] && !staged[y] && overlaps(inter[x], inter[y])) staged[x] = true;
    }
    const sl_buffer_ref att = at.out;
    const bool att_dead = mh != nullptr && dead_after(d, i + used, att);
    AttentionArgs a{fptr(d, sq.in[0]), fptr(d, sk.in[0]), fptr(d, sv.in[0]), fptr(d, cache),
                    att_dead ? nullptr : fptr(d, att), B, ap.layers, ap.layer, H, Hkv, S, ap.past_len, D,
                    ap.max_seq, ap.scale, dyn_of(d, at)};
    if (paged) set_paged(d, *paged, &a);
    // The prefill form writes its rotated q to a workspace area and takes
    // no other live intermediate: a live rotated q (the last layer's, which
    // nothing overwrites before the submission ends) is staged there and
    // copied to its place like the decode form's.
    if (attention_fused_prefill(a)) {
        if (live[0] || live[1] || live[2] || live[4]) return 0;
        staged[3] = live[3];
    }
    // Workspace: the decode partials (prefill: the rotated q), the mirror of
    // the merged heads, then the staged intermediates.
    const Workspace ws{d->workspace, d->workspace_floats};
    const uint64_t mirror_at = (attention_fused_workspace_floats(a) + 63) / 64 * 64;
    // The output projection is chained (it reads the mirror, not MergeHeads'
    // output) only for decode (at most 16 rows, the fused GEMV's) and when
    // the mirror fits; otherwise it runs on its own and reads MergeHeads'
    // output, which must then be written.
    const Logged* mm = mh && i + used < n ? &d->log[i + used] : nullptr;
    const bool chain = mm && mm->plan.code == SL_OP_MATMUL_NT && same_ref(mm->in[0], mh->out) &&
                       mfma_weight(d, *mm, 1) && mm->plan.batch * mm->plan.m == B * S && mm->plan.k == H * D &&
                       B * S <= 16 && mirror_at + B * S * H * D <= ws.floats;
    const bool merged_needed = mh != nullptr && !dead_after(d, i + used, mh->out, chain ? i + used : SIZE_MAX);
    // outputs of the merge kernel: no overlap with the cache, or with each other
    if (overlaps(att, cache_ref) || (mh && overlaps(mh->out, cache_ref)) ||
        (mh && !att_dead && merged_needed && overlaps(att, mh->out) && !same_ref(att, mh->out)))
        return 0;
    a.positions = uptr(d, rq.in[1]);
    a.theta = rq.plan.theta;
    a.rope_variant = rq.plan.rope_variant;
    a.merged = merged_needed ? fptr(d, mh->out) : nullptr;
    // the Rope table: computed once per submission for these positions,
    // again only if a command since has written the positions buffer
    const uint64_t tokens = B * S;
    if (tokens * D <= kRopeTableFloats) {
        auto& rt = d->rope;
        bool fresh = rt.valid && same_ref(rt.pos, rq.in[1]) && rt.theta == rq.plan.theta && rt.head_dim == D &&
                     rt.tokens == tokens;
        for (size_t x = rt.at; fresh && x < i; ++x)
            if (overlaps(d->log[x].out, rt.pos)) fresh = false;
        if (!fresh) {
            const hipError_t te = launch_rope_sincos(a.positions, tokens, D, rq.plan.theta, d->rope_tab, d->stream);
            if (te != hipSuccess) {
                *err = te;
                return 1;
            }
            rt.valid = true;
            rt.pos = rq.in[1];
            rt.theta = rq.plan.theta;
            rt.head_dim = D;
            rt.tokens = tokens;
            rt.at = i;
        }
        a.rope_table = d->rope_tab;
    }
    uint64_t stage_at = mirror_at + (B * S * H * D + 63) / 64 * 64;
    float* stage[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
    float** const inter_ptr[5] = {&a.q_split, &a.k_split, &a.v_split, &a.q_rot, &a.k_rot};
    for (int x = 0; x < 5; ++x) {
        if (!live[x]) continue;
        if (staged[x]) {
            if (stage_at + inter[x].len > ws.floats) return 0;
            stage[x] = ws.data + stage_at;
            stage_at += (inter[x].len + 63) / 64 * 64;
            *inter_ptr[x] = stage[x];
        } else {
            *inter_ptr[x] = fptr(d, inter[x]);
        }
    }

    // the output projection (and its residual Add) reading the mirror
    if (chain) a.mirror = ws.data + mirror_at;
    hipError_t e = launch_attention_fused(a, ws, d->stream);
    if (e == hipErrorNotSupported) return 0;
    if (e != hipSuccess) {
        *err = e;
        return used;
    }
    // staged intermediates to their place: the ranges that the unit's later
    // commands (the other intermediates, the attention output, MergeHeads)
    // leave holding them, before the chained projection writes anything
    const size_t unit_end = i + (mh != nullptr ? 7 : 6);
    for (int x = 0; x < 5 && e == hipSuccess; ++x) {
        if (stage[x] == nullptr) continue;
        std::vector<std::pair<uint64_t, uint64_t>> keep{{inter[x].offset, inter[x].offset + inter[x].len}};
        for (size_t j = i + x + 1; j < unit_end; ++j) {
            const sl_buffer_ref& o = d->log[j].out;
            if (o.buffer != inter[x].buffer || o.len == 0) continue;
            std::vector<std::pair<uint64_t, uint64_t>> rest;
            for (const auto& iv : keep) {
                if (o.offset > iv.first) rest.push_back({iv.first, o.offset < iv.second ? o.offset : iv.second});
                if (o.offset + o.len < iv.second)
                    rest.push_back({o.offset + o.len > iv.first ? o.offset + o.len : iv.first, iv.second});
            }
            keep.clear();
            for (const auto& iv : rest)
                if (iv.first < iv.second) keep.push_back(iv);
        }
        for (const auto& iv : keep) {
            sl_buffer_ref part = inter[x];
            part.offset = iv.first;
            part.len = iv.second - iv.first;
            e = launch_copy(stage[x] + (iv.first - inter[x].offset), fptr(d, part), part.len, d->stream);
            if (e != hipSuccess) break;
        }
    }
    if (e != hipSuccess) {
        *err = e;
        return used;
    }
    if (chain) {
        QuantWeight w = weight_ref(d, mm->in[1], mm->plan.quant[1]).quant;
        QgemvFused f{};
        f.a = a.mirror;
        f.w[0] = &w;
        f.out[0] = fptr(d, mm->out);
        f.nseg = 1;
        f.m = B * S;
        f.epilogue = kFusedPlain;
        size_t extra = 1;
        if (i + used + 1 < n) {
            const Logged& ad = d->log[i + used + 1];
            const int other = residual_port(ad, mm->out, B * S * w.n, nullptr, 0);
            if (other >= 0) {
                f.epilogue = kFusedResidual;
                f.resid[0] = fptr(d, ad.in[other]);
                f.out2[0] = fptr(d, ad.out);
                extra = 2;
            }
        }
        e = launch_qgemv_fused(f, d->stream);
        if (e == hipErrorNotSupported) {
            // run the projection on its own, from the mirror
            e = launch_qmatmul(a.mirror, w, f.out[0], B * S, ws.after(mirror_at + B * S * H * D), d->stream);
            extra = 1;
        }
        used += extra;
    }
    *err = e;
    d->stats.fused_commands += used;
    return used;
}

// Silu(x) -> t then Mul(t, u) -> out as one pass, out = silu(x) * u, when t
// is dead after the Mul (every element overwritten before any read): the
// product's two IEEE multiplies are the unfused ones (a * b == b * a), so
// the result is bit-identical and t is never written. The outputs of both
// commands are disjoint from their inputs (validated); x may be out itself.
size_t try_fuse_silu_mul(Device* d, size_t i, hipError_t* err) {
    if (i + 2 > d->log.size()) return 0;
    const Logged &sc = d->log[i], &mc = d->log[i + 1];
    if (sc.plan.code != SL_OP_SILU || mc.plan.code != SL_OP_MUL || sc.plan.len != mc.plan.len) return 0;
    const sl_buffer_ref& t = sc.out;
    const int other = same_ref(mc.in[0], t) ? 1 : same_ref(mc.in[1], t) ? 0 : -1;
    if (other < 0) return 0;
    const sl_buffer_ref &x = sc.in[0], &u = mc.in[other], &out = mc.out;
    if (overlaps(u, t) || (overlaps(out, x) && !same_ref(out, x)) || !dead_after(d, i + 1, t, i + 1)) return 0;
    *err = launch_silu_mul(fptr(d, x), fptr(d, u), fptr(d, out), sc.plan.len, d->stream);
    d->stats.fused_commands += 2;
    return 2;
}

hipError_t run_log(Device* d) {
    d->rope.valid = false;
    for (size_t i = 0; i < d->log.size();) {
        size_t used = 0;
        hipError_t e = hipSuccess;
        if (d->options & SL_HIP_OPT_FUSION) {
            used = try_fuse_attention(d, i, &e);
            if (used == 0 && e == hipSuccess) used = try_fuse(d, i, &e);
            if (used == 0 && e == hipSuccess) used = try_fuse_silu_mul(d, i, &e);
        }
        if (e != hipSuccess) return e;
        if (used == 0) {
            const Logged& c = d->log[i];
            e = launch(d, c.plan, c.in, &c.out, dyn_of(d, c),
                       Workspace{d->workspace, d->workspace_floats});
            if (e != hipSuccess) return e;
            used = 1;
        }
        i += used;
    }
    return hipSuccess;
}

void drop_graphs(Device* d) {
    for (GraphEntry& g : d->graphs) {
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
        if (g.graph) (void)hipGraphDestroy(g.graph);
    }
    d->graphs.clear();
    d->last_graph = SIZE_MAX;
    d->prev_key.clear();
}

// Everything that decides which kernels a submission launches, with what
// arguments: the commands (past_len aside) and the submission options.
void build_key(Device* d) {
    std::vector<uint64_t>& k = d->key;
    k.clear();
    k.push_back(d->options);
    auto f = [](float x) {
        uint32_t u;
        std::memcpy(&u, &x, 4);
        return static_cast<uint64_t>(u);
    };
    for (const Logged& c : d->log) {
        const Plan& p = c.plan;
        k.insert(k.end(), {p.code, p.rows, p.cols, p.hidden, p.batch, p.batch_a, p.batch_b, p.m, p.k, p.n, p.heads,
                           p.kv_heads, p.seq, p.head_dim, p.layers, p.layer, p.max_seq,
                           reads_past(p.code) ? 0 : p.past_len, p.seq_len, p.vocab, p.inter, p.out_features, p.len,
                           f(p.eps), f(p.theta), f(p.factor), f(p.scale), p.rope_variant,
                           static_cast<uint64_t>(static_cast<int64_t>(p.state_index)), c.n_in,
                           static_cast<uint64_t>(static_cast<int64_t>(c.dyn_slot))});
        for (size_t i = 0; i < kMaxInputs; ++i) {
            const QuantOperand& q = p.quant[i];
            k.insert(k.end(), {static_cast<uint64_t>(q.present), q.format, q.group, q.n, q.k});
        }
        for (uint32_t i = 0; i < c.n_in; ++i) k.insert(k.end(), {c.in[i].buffer, c.in[i].offset, c.in[i].len});
        k.insert(k.end(), {c.out.buffer, c.out.offset, c.out.len});
    }
}

// FNV-style over 8 interleaved lanes: one chain of dependent multiplies
// per lane rather than one for the whole key (tens of thousands of words
// per decode step).
uint64_t key_hash(const std::vector<uint64_t>& k) {
    constexpr size_t kLanes = 8;
    uint64_t h[kLanes];
    for (size_t l = 0; l < kLanes; ++l) h[l] = 1469598103934665603ull + l;
    const size_t n = k.size(), body = n / kLanes * kLanes;
    for (size_t i = 0; i < body; i += kLanes)
        for (size_t l = 0; l < kLanes; ++l) h[l] = (h[l] ^ k[i + l]) * 1099511628211ull;
    for (size_t i = body; i < n; ++i) h[0] = (h[0] ^ k[i]) * 1099511628211ull;
    uint64_t r = n;
    for (size_t l = 0; l < kLanes; ++l) r = (r ^ h[l]) * 1099511628211ull;
    return r;
}

// Enqueues the logged commands; the log is empty afterwards either way.
hipError_t submit(Device* d) {
    if (d->log.empty()) return hipSuccess;
    hipError_t e = hipSuccess;
    // One past_len slot per logged command that reads it; the log never
    // exceeds kLogFlushLength commands, the array's size (allocated with the
    // device, so a submission allocates nothing for it).
    uint32_t slots = 0;
    for (Logged& c : d->log) c.dyn_slot = reads_past(c.plan.code) ? static_cast<int32_t>(slots++) : -1;
    d->dyn_values.clear();
    for (const Logged& c : d->log)
        if (c.dyn_slot >= 0) d->dyn_values.push_back(static_cast<uint32_t>(c.plan.past_len));
    if (slots) e = launch_set_words(d->dyn, d->dyn_values.data(), slots, d->stream);

    d->stats.submissions += 1;
    d->stats.commands += d->log.size();
    build_key(d);
    // A decode loop submits the same commands every step: the entry the
    // previous submission used is tried first, by its key alone.
    GraphEntry* hit = nullptr;
    uint64_t hash = 0;
    if (d->last_graph < d->graphs.size() && d->graphs[d->last_graph].key == d->key) {
        hit = &d->graphs[d->last_graph];
    } else {
        hash = key_hash(d->key);
        for (GraphEntry& g : d->graphs)
            if (g.hash == hash && g.key == d->key) hit = &g;
    }
    if (e != hipSuccess) {
        // nothing more
    } else if (hit) {
        hit->last_use = ++d->use_clock;
        d->last_graph = static_cast<size_t>(hit - d->graphs.data());
        e = hipGraphLaunch(hit->exec, d->stream);
        d->stats.graph_replays += 1;
    } else if ((d->options & SL_HIP_OPT_GRAPHS) && d->key == d->prev_key) {
        // Seen twice in a row: capture it.
        GraphEntry g;
        bool captured = false;
        if (hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal) == hipSuccess) {
            const hipError_t run = run_log(d);
            const hipError_t end = hipStreamEndCapture(d->stream, &g.graph);
            if (run == hipSuccess && end == hipSuccess && g.graph &&
                hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0) == hipSuccess)
                captured = true;
        }
        if (captured) {
            if (d->graphs.size() >= kGraphCacheSize) {
                size_t lru = 0;
                for (size_t i = 1; i < d->graphs.size(); ++i)
                    if (d->graphs[i].last_use < d->graphs[lru].last_use) lru = i;
                (void)hipGraphExecDestroy(d->graphs[lru].exec);
                (void)hipGraphDestroy(d->graphs[lru].graph);
                d->graphs.erase(d->graphs.begin() + static_cast<std::ptrdiff_t>(lru));
            }
            g.key = d->key;
            g.hash = hash;
            g.last_use = ++d->use_clock;
            d->graphs.push_back(g);
            d->last_graph = d->graphs.size() - 1;
            e = hipGraphLaunch(d->graphs.back().exec, d->stream);
            d->stats.graph_captures += 1;
        } else {
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
            if (g.graph) (void)hipGraphDestroy(g.graph);
            (void)hipGetLastError();
            e = run_log(d);
        }
    } else {
        e = run_log(d);
    }
    std::swap(d->prev_key, d->key);
    d->log.clear();
    return e;
}

// The device workspace size: SL_HIP_WORKSPACE_BYTES when set (at least
// 64 KiB, rounded up to 256 bytes), else 512 MiB. Fused paths that do not
// fit a smaller workspace fall back to their unfused kernels.
uint64_t workspace_bytes_setting() {
    const char* v = std::getenv("SL_HIP_WORKSPACE_BYTES");
    if (v == nullptr || *v == 0) return kWorkspaceBytes;
    char* end = nullptr;
    const unsigned long long n = std::strtoull(v, &end, 10);
    if (end == v || *end != 0) return kWorkspaceBytes;
    const uint64_t lo = 64ull << 10;
    const uint64_t b = n < lo ? lo : n;
    return (b + 255) / 256 * 256;
}

sl_status flush(Device* d) {
    const hipError_t e = submit(d);
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
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
    // Every kernel file's code object now rather than inside the first
    // submission that needs it (about 5 ms of a first 8B prefill). A file
    // that does not load here fails at its first launch with that error.
    (void)slhip::preload_code();
    (void)hipGetLastError();
    const uint64_t ws_bytes = slhip::workspace_bytes_setting();
    if (hipMalloc(reinterpret_cast<void**>(&d->workspace), ws_bytes) != hipSuccess) {
        (void)hipStreamDestroy(d->stream);
        delete d;
        return SL_ERR_OUT_OF_MEMORY;
    }
    d->workspace_floats = ws_bytes / 4;
    if (hipMalloc(reinterpret_cast<void**>(&d->rope_tab), slhip::kRopeTableFloats * 4) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&d->dyn), slhip::kLogFlushLength * sizeof(uint32_t)) != hipSuccess) {
        (void)hipGetLastError();
        if (d->rope_tab) (void)hipFree(d->rope_tab);
        (void)hipFree(d->workspace);
        (void)hipStreamDestroy(d->stream);
        delete d;
        return SL_ERR_OUT_OF_MEMORY;
    }
    d->id_scratch.resize(slhip::kIdScratchElements);
    // The static scratch array's address on this GPU (current here); kept
    // per device, and a failed lookup leaves only the no-allocation entry
    // point unavailable.
    if (slhip::static_scratch_address(ordinal, &d->static_scratch) != hipSuccess) {
        (void)hipGetLastError();
        d->static_scratch = nullptr;
    }
    *out = d;
    return SL_OK;
}

void sl_hip_device_destroy(sl_hip_device* d) {
    if (d == nullptr) return;
    (void)hipSetDevice(d->ordinal);
    (void)slhip::flush(d);
    (void)hipStreamSynchronize(d->stream);
    slhip::drop_graphs(d);
    if (d->dyn) (void)hipFree(d->dyn);
    for (auto& b : d->buffers) {
        if (b.base) (void)hipFree(b.base);
        if (b.tiles) (void)hipFree(b.tiles);
    }
    if (d->workspace) (void)hipFree(d->workspace);
    if (d->rope_tab) (void)hipFree(d->rope_tab);
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
    if (!slhip::device_limits(plan, d->workspace_floats, &err)) return d->fail(err);
    if (plan.code == SL_OP_GATHER && !slhip::gather_ids_in_range(d, inputs[1], plan.vocab, &err))
        return d->fail(err);
    if (plan.state_index >= 0)
        if (const sl_paged_kv* kv = d->paged_of(inputs[plan.state_index].buffer))
            if (!slhip::check_paged_command(d, plan, *kv, &err)) return d->fail(err);
    slhip::Logged c;
    c.plan = plan;
    c.n_in = static_cast<uint32_t>(n_inputs);
    for (size_t i = 0; i < n_inputs; ++i) c.in[i] = inputs[i];
    if (n_outputs) c.out = outputs[0];
    d->log.push_back(c);
    if (d->log.size() >= slhip::kLogFlushLength) return slhip::flush(d);
    return SL_OK;
}

sl_status sl_hip_dispatch_noalloc(sl_hip_device* d, const sl_op* op, const sl_buffer_ref* inputs,
                                  const sl_value* input_values, size_t n_inputs, const sl_buffer_ref* outputs,
                                  const sl_value* output_values, size_t n_outputs, const uint32_t* scalars,
                                  size_t n_scalars) {
    slhip::Plan plan;
    Error err;
    if (!slhip::validate_dispatch(*d, *op, inputs, input_values, n_inputs, outputs, output_values, n_outputs,
                                  scalars, n_scalars, &plan, &err))
        return d->fail(err);
    if (!slhip::device_limits(plan, slhip::kStaticScratchFloats, &err)) return d->fail(err);
    if (!d->log.empty())
        return d->fail(Error::execution("commands are still logged: submit them before sl_hip_dispatch_noalloc"));
    if (d->static_scratch == nullptr)
        return d->fail(Error::execution("the static scratch array is not available on this device"));
    if (plan.code == SL_OP_GATHER && !slhip::gather_ids_in_range(d, inputs[1], plan.vocab, &err))
        return d->fail(err);
    sl_buffer_ref out{};
    if (n_outputs) out = outputs[0];
    // past_len reaches the kernels as the scalar itself (no device word)
    const hipError_t e =
        slhip::launch(d, plan, inputs, &out, nullptr,
                      slhip::Workspace{d->static_scratch, slhip::kStaticScratchFloats});
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
}

sl_status sl_hip_paged_attention(sl_hip_device* d, const sl_op* op, const sl_buffer_ref* q,
                                 const sl_buffer_ref* k_new, const sl_buffer_ref* v_new, const sl_buffer_ref* out,
                                 uint32_t batch, const sl_paged_kv* kv) {
    using slhip::Error;
    if (op == nullptr || q == nullptr || k_new == nullptr || v_new == nullptr || out == nullptr || kv == nullptr)
        return d->fail(Error::execution("paged attention received a null argument"));
    if (op->code != SL_OP_CAUSAL_ATTENTION) return d->fail(Error::unsupported_op(op->code));
    const uint64_t H = op->heads, Hkv = op->kv_heads, D = op->head_dim, B = batch;
    if (Hkv == 0 || H == 0 || H % Hkv != 0) return d->fail(Error::execution("heads must be a multiple of kv_heads"));
    if (D == 0 || D % 64 != 0 || D > 256)
        return d->fail(Error::unimplemented("paged attention needs head_dim a multiple of 64 up to 256"));
    if (H / Hkv > 16) return d->fail(Error::unimplemented("paged attention takes at most 16 query heads per KV head"));
    if (kv->layers == 0 || op->layer >= kv->layers) return d->fail(Error::execution("layer is out of range"));
    // ports: f32 ranges of the stated sizes, the output disjoint from the inputs
    const struct {
        const sl_buffer_ref* r;
        uint64_t len;
    } ports[4] = {{q, B * H * D}, {k_new, B * Hkv * D}, {v_new, B * Hkv * D}, {out, B * H * D}};
    for (const auto& pt : ports) {
        const sl_buffer_ref& r = *pt.r;
        if (r.buffer >= d->buffers.size() || d->buffers[r.buffer].desc.kind != SL_BUFFER_F32)
            return d->fail(Error::invalid_buffer(r.buffer));
        if (r.len != pt.len) return d->fail(Error::execution("paged attention port has the wrong length"));
        if (r.offset > d->buffers[r.buffer].desc.elements || r.len > d->buffers[r.buffer].desc.elements - r.offset)
            return d->fail(Error::invalid_range(r.buffer, r.offset, r.len));
    }
    for (int i = 0; i < 3; ++i)
        if (slhip::overlaps(*ports[i].r, *out))
            return d->fail(Error::execution("a command output aliases an overlapping input range"));
    Error err;
    if (!slhip::check_paged_buffers(d, *kv, Hkv, D, &err)) return d->fail(err);
    for (const auto& pt : ports)
        if (pt.r->buffer == kv->pool)
            return d->fail(Error::execution("a command output aliases an overlapping input range"));
    if (!slhip::check_paged_tables(d, *kv, B, &err)) return d->fail(err);
    const slhip::Buffer& tb = d->buffers[kv->block_table];
    const slhip::Buffer& lb = d->buffers[kv->seq_lens];
    if (B == 0) return SL_OK;  // an empty batch: nothing to read or append
    if (slhip::flush(d) != SL_OK) return d->last.status;
    slhip::PagedAttentionArgs a{};
    a.q = slhip::fptr(d, *q);
    a.k_new = slhip::fptr(d, *k_new);
    a.v_new = slhip::fptr(d, *v_new);
    a.pool = static_cast<float*>(d->buffers[kv->pool].ptr);
    a.out = slhip::fptr(d, *out);
    a.block_table = static_cast<const uint32_t*>(tb.ptr);
    a.seq_lens = static_cast<const uint32_t*>(lb.ptr);
    a.batch = B;
    a.layers = kv->layers;
    a.layer = op->layer;
    a.heads = H;
    a.kv_heads = Hkv;
    a.head_dim = D;
    a.num_pages = kv->num_pages;
    a.page_size = kv->page_size;
    a.pages_per_seq = kv->pages_per_seq;
    a.scale = op->scale;
    if (slhip::paged_attention_workspace_floats(a) > d->workspace_floats)
        return d->fail(Error::unimplemented("paged attention partials exceed the device workspace"));
    const hipError_t e = slhip::launch_paged_attention(
        a, slhip::Workspace{d->workspace, d->workspace_floats}, d->stream);
    if (e == hipErrorNotSupported) return d->fail(Error::unimplemented("paged attention shape is not supported"));
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
}

sl_status sl_hip_synchronize(sl_hip_device* d) {
    if (slhip::flush(d) != SL_OK) return d->last.status;
    hipError_t e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
}

sl_status sl_hip_bind_paged_state(sl_hip_device* d, uint32_t state, const sl_paged_kv* kv) {
    using slhip::Error;
    if (state >= d->buffers.size() || d->buffers[state].desc.kind != SL_BUFFER_F32)
        return d->fail(Error::invalid_buffer(state));
    if (kv != nullptr) {
        Error err;
        if (!slhip::check_paged_buffers(d, *kv, 0, 0, &err)) return d->fail(err);
        if (kv->pool == state) return d->fail(Error::execution("a State cannot be bound to itself as a page pool"));
    }
    // logged commands read the previous binding; graphs hold its addresses
    if (slhip::flush(d) != SL_OK) return d->last.status;
    slhip::drop_graphs(d);
    auto& v = d->paged_states;
    for (size_t i = 0; i < v.size(); ++i)
        if (v[i].first == state) {
            v.erase(v.begin() + static_cast<std::ptrdiff_t>(i));
            break;
        }
    if (kv != nullptr) v.push_back({state, *kv});
    return SL_OK;
}

sl_status sl_hip_paged_store(sl_hip_device* d, const sl_paged_kv* kv, uint32_t row, uint32_t state, uint32_t index,
                             uint32_t max_seq, uint32_t kv_heads, uint32_t head_dim, uint32_t length) {
    using slhip::Error;
    if (kv == nullptr) return d->fail(Error::execution("paged store received a null argument"));
    Error err;
    if (!slhip::check_paged_buffers(d, *kv, kv_heads, head_dim, &err)) return d->fail(err);
    if (state >= d->buffers.size() || d->buffers[state].desc.kind != SL_BUFFER_F32)
        return d->fail(Error::invalid_buffer(state));
    const uint64_t row_floats = static_cast<uint64_t>(kv_heads) * head_dim;
    const uint64_t per_index = static_cast<uint64_t>(kv->layers) * 2 * max_seq * row_floats;
    if (row_floats == 0 || row_floats % 4 != 0 || per_index == 0 ||
        d->buffers[state].desc.elements % per_index != 0 || index >= d->buffers[state].desc.elements / per_index)
        return d->fail(Error::execution("State buffer size does not match [batch, layers, 2, max_seq, kv_heads, "
                                        "head_dim]"));
    if (length > max_seq) return d->fail(Error::execution("paged store length exceeds max_seq"));
    const slhip::Buffer& tb = d->buffers[kv->block_table];
    if (tb.desc.elements < (static_cast<uint64_t>(row) + 1) * kv->pages_per_seq)
        return d->fail(Error::execution("block table or lengths buffer is too small for the batch"));
    if (length != 0) {
        const uint64_t last = (static_cast<uint64_t>(length) - 1) / kv->page_size;
        if (last >= kv->pages_per_seq) return d->fail(Error::execution("paged KV length exceeds the row's block table"));
        for (uint64_t pi = 0; pi <= last; ++pi)
            if (tb.mirror[static_cast<uint64_t>(row) * kv->pages_per_seq + pi] >= kv->num_pages)
                return d->fail(Error::execution("page id out of range"));
    }
    if (slhip::flush(d) != SL_OK) return d->last.status;
    const hipError_t e = slhip::launch_paged_store(
        static_cast<const float*>(d->buffers[state].ptr), static_cast<float*>(d->buffers[kv->pool].ptr),
        static_cast<const uint32_t*>(tb.ptr) + static_cast<uint64_t>(row) * kv->pages_per_seq, index, kv->layers,
        max_seq, row_floats, kv->num_pages, kv->page_size, length, d->stream);
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
}

sl_status sl_hip_submit(sl_hip_device* d) { return slhip::flush(d); }

sl_status sl_hip_set_options(sl_hip_device* d, uint32_t options) {
    if (slhip::flush(d) != SL_OK) return d->last.status;
    d->options = options & (SL_HIP_OPT_FUSION | SL_HIP_OPT_GRAPHS);
    d->prev_key.clear();
    return SL_OK;
}

void sl_hip_get_stats(const sl_hip_device* d, sl_hip_stats* out) { *out = d->stats; }

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
    // The same binding again (Engine build binds every quantized Param of
    // each program it builds): nothing changes. The tile copy is already
    // current, since re-uploads of the payload or scales refresh it.
    if (pb.tiles != nullptr && pb.desc.quantized && pb.scales == scales && pb.desc.qformat == qformat &&
        pb.desc.group_size == group_size && pb.desc.qn == n && pb.desc.qk == k)
        return SL_OK;
    // Logged commands read the old binding; the graphs hold its tile address.
    if (slhip::flush(d) != SL_OK) return d->last.status;
    slhip::drop_graphs(d);
    const slhip::QuantLayout layout = slhip::quant_layout_for(qformat, n, k, group_size);
    const uint64_t code_bytes = slhip::quant_tile_bytes(qformat, n, k, layout);
    const uint64_t scale_offset = (code_bytes + 255) / 256 * 256;
    const uint64_t scale_floats = slhip::quant_tile_scale_floats(n, k, group_size, layout);
    const uint64_t bytes = scale_floats ? scale_offset + scale_floats * 4 : code_bytes;
    if (pb.tiles) {
        (void)hipStreamSynchronize(d->stream);
        (void)hipFree(pb.tiles);
        pb.tiles = nullptr;
        pb.tile_scales = nullptr;
    }
    if (bytes != 0) {
        if (hipMalloc(reinterpret_cast<void**>(&pb.tiles), bytes) != hipSuccess) {
            (void)hipGetLastError();
            pb.tiles = nullptr;
            return d->fail(Error::out_of_memory(bytes / 4));
        }
        if (scale_floats) pb.tile_scales = reinterpret_cast<float*>(pb.tiles + scale_offset);
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
    if (e == hipSuccess && pb.tile_scales)
        e = slhip::launch_scale_repack(static_cast<const float*>(d->buffers[scales].ptr), pb.tile_scales, n, k,
                                       group_size, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
}

void* sl_hip_stream(const sl_hip_device* d) { return d->stream; }

}  // extern "C"

sl_status slhip_fail_execution(sl_hip_device* d, const char* message) {
    return d->fail(Error::execution(message));
}

extern "C" {

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
