// Host-side launchers of the gfx950 kernels. Every launcher enqueues on
// `stream` and returns the launch status; shapes have already been validated.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "starlight_hip.h"

namespace slhip {

// Device-owned scratch passed to kernels that need it: partial results and
// intermediates.
struct Workspace {
    float* data;
    uint64_t floats;

    // The part of `data` after the first `used` floats.
    Workspace after(uint64_t used) const {
        Workspace w = *this;
        used = (used + 63) / 64 * 64;  // keep 256-byte alignment
        w.data = used < floats ? data + used : data + floats;
        w.floats = used < floats ? floats - used : 0;
        return w;
    }
};

// ---- elementwise (reference/elementwise.rs) ----
// Each kernel file's code object, loaded ahead of its first launch (HIP
// loads one at the first use of any of its kernels); preload_code loads
// them all and returns the first error.
hipError_t load_code_attention();
hipError_t load_code_elementwise();
hipError_t load_code_layout();
hipError_t load_code_matmul();
hipError_t load_code_norm_softmax();
hipError_t load_code_qgemm_mfma();
hipError_t load_code_qgemv_fused();
hipError_t load_code_qgemv_mfma();
hipError_t load_code_qmatmul();
hipError_t load_code_rope();
inline hipError_t preload_code() {
    hipError_t (*const loads[])() = {load_code_attention, load_code_elementwise, load_code_layout,
                                     load_code_matmul,    load_code_norm_softmax, load_code_qgemm_mfma,
                                     load_code_qgemv_fused, load_code_qgemv_mfma, load_code_qmatmul,
                                     load_code_rope};
    hipError_t first = hipSuccess;
    for (auto load : loads) {
        const hipError_t e = load();
        if (first == hipSuccess) first = e;
    }
    return first;
}

hipError_t launch_add(const float* a, const float* b, float* out, uint64_t n, hipStream_t s);
hipError_t launch_mul(const float* a, const float* b, float* out, uint64_t n, hipStream_t s);
hipError_t launch_scale(const float* x, float* out, uint64_t n, float factor, hipStream_t s);
hipError_t launch_silu(const float* x, float* out, uint64_t n, hipStream_t s);
hipError_t launch_fill_zero(float* out, uint64_t n, hipStream_t s);
// dst[i] = src[i] (bit copies; the ranges must not overlap).
hipError_t launch_copy(const float* src, float* dst, uint64_t n, hipStream_t s);

// dst[0..count) = values, through kernel arguments (no host buffer lifetime,
// no memset node when captured).
hipError_t launch_set_words(uint32_t* dst, const uint32_t* values, uint64_t count, hipStream_t s);

// Launchers whose kernels read past_len also take `dyn`: when set, the
// kernels read past_len from dyn[0] at run time instead of the argument.
// Their launch geometry never depends on past_len, so a captured launch is
// valid for any length.

// ---- norm / softmax (reference/norm.rs, reference/softmax.rs) ----
hipError_t launch_rms_norm(const float* x, const float* w, float* out, uint64_t rows, uint64_t hidden,
                           float eps, hipStream_t s);
hipError_t launch_softmax(const float* x, float* out, uint64_t rows, uint64_t cols, bool causal,
                          uint64_t seq, uint64_t past_len, const uint32_t* dyn, hipStream_t s);

// ---- rope (reference/rope.rs) ----
hipError_t launch_rope(const float* x, const uint32_t* positions, float* out, uint64_t batch,
                       uint64_t heads, uint64_t seq, uint64_t head_dim, float theta, bool interleaved,
                       hipStream_t s);

// ---- layout (reference/layout.rs, attention.rs kv_append) ----
hipError_t launch_gather(const float* table, const uint32_t* ids, float* out, uint64_t rows,
                         uint64_t hidden, hipStream_t s);
hipError_t launch_last_token(const float* in, float* out, uint64_t batch, uint64_t seq, uint64_t hidden,
                             uint64_t seq_len, hipStream_t s);
hipError_t launch_heads_permute(const float* in, float* out, uint64_t batch, uint64_t seq,
                                uint64_t heads, uint64_t head_dim, bool split, hipStream_t s);
hipError_t launch_kv_append(const float* k, const float* v, float* cache, uint64_t batch,
                            uint64_t layers, uint64_t layer, uint64_t kv_heads, uint64_t head_dim,
                            uint64_t max_seq, uint64_t past_len, uint64_t seq, const uint32_t* dyn,
                            hipStream_t s);

// ---- attention (reference/attention.rs causal_attention, kv_append included) ----
struct AttentionArgs {
    const float* q;
    const float* k_new;
    const float* v_new;
    float* cache;
    float* out;
    uint64_t batch, layers, layer, heads, kv_heads, seq, past_len, head_dim, max_seq;
    float scale;
    const uint32_t* dyn;  // device copy of past_len read by the kernels, or null
    // Fused form (launch_attention_fused): q / k_new / v_new are the
    // projections before SplitHeads, [batch, seq, heads * head_dim], and are
    // rotated by Rope at `positions` inside the kernel; `out` (the attention
    // output, may be null), `merged` (MergeHeads of it, may be null) and
    // `mirror` (a copy of merged in the workspace, may be null) are written.
    const uint32_t* positions = nullptr;
    float theta = 0.f;
    uint32_t rope_variant = 0;
    float* merged = nullptr;
    float* mirror = nullptr;
    // Fused form, when a later command reads them: the SplitHeads outputs
    // [batch, heads, seq, head_dim] of q / k / v and the Rope outputs of q / k
    // (same layout), each written when non-null.
    float* q_split = nullptr;
    float* k_split = nullptr;
    float* v_split = nullptr;
    float* q_rot = nullptr;
    float* k_rot = nullptr;
    // Fused form: the Rope sine / cosine table of these positions
    // (launch_rope_sincos), or null to compute it in every block.
    const float* rope_table = nullptr;
    // Decode form over a paged cache, when block_table is set: `cache` is
    // the page pool [layers][num_pages][2][page_size][kv_heads][head_dim],
    // row b has seq_lens[b] cached positions (past_len and max_seq are not
    // read: the capacity is pages_per_seq * page_size), position j lives in
    // page block_table[b * pages_per_seq + j / page_size].
    const uint32_t* block_table = nullptr;
    const uint32_t* seq_lens = nullptr;
    uint32_t num_pages = 0, page_size = 0, pages_per_seq = 0;
};
// Rope angles' sine and cosine for `tokens` positions: table[t * head_dim +
// pair] = sin, table[t * head_dim + head_dim / 2 + pair] = cos, from f64
// pow / sin / cos rounded once (reference/rope.rs:32-35).
hipError_t launch_rope_sincos(const uint32_t* positions, uint64_t tokens, uint64_t head_dim, float theta,
                              float* table, hipStream_t s);
// Floats of the static per-GPU scratch array of the no-allocation entry
// point (SL_HIP_STATIC_SCRATCH_BYTES).
constexpr uint64_t kStaticScratchFloats = SL_HIP_STATIC_SCRATCH_BYTES / 4;
// Its address on device `ordinal`, which must be the current device at the
// first call for that ordinal (hipGetSymbolAddress, cached per ordinal).
hipError_t static_scratch_address(int ordinal, float** out);

// Appends k_new / v_new to the cache and computes the attention output.
hipError_t launch_attention(const AttentionArgs& a, const Workspace& ws, hipStream_t s);
// SplitHeads x3 + Rope x2 + CausalAttention (+ MergeHeads) as the two decode
// launches; hipErrorNotSupported (nothing launched) for shapes the decode
// kernel does not take. `mirror` must lie in `ws` past the first
// attention_workspace_floats(a) floats.
hipError_t launch_attention_fused(const AttentionArgs& a, const Workspace& ws, hipStream_t s);
uint64_t attention_workspace_floats(const AttentionArgs& a);
// Whether launch_attention_fused takes the prefill form for this shape
// (more query rows per KV head than the decode kernel serves), and the
// workspace floats its kernels use before any caller area: the decode
// partials, or the prefill form's rotated q.
bool attention_fused_prefill(const AttentionArgs& a);
uint64_t attention_fused_workspace_floats(const AttentionArgs& a);

// Decode attention over a paged KV cache (one new token per row): row b has
// seq_lens[b] cached positions; its new K/V row is appended at position
// seq_lens[b] and its queries attend to positions 0..seq_lens[b]. The pool is
// [layers][num_pages][2][page_size][kv_heads][head_dim]; position j of row b
// lives in page block_table[b * pages_per_seq + j / page_size], slot
// j % page_size. q / out [batch, heads, 1, head_dim]; k_new / v_new
// [batch, kv_heads, 1, head_dim]. page_size must be a multiple of 16 and the
// shapes those of the decode kernel (else hipErrorNotSupported, nothing
// launched). The caller checks that the table and lengths stay in range.
struct PagedAttentionArgs {
    const float* q;
    const float* k_new;
    const float* v_new;
    float* pool;
    float* out;
    const uint32_t* block_table;
    const uint32_t* seq_lens;
    uint64_t batch, layers, layer, heads, kv_heads, head_dim;
    uint32_t num_pages, page_size, pages_per_seq;
    float scale;
};
hipError_t launch_paged_attention(const PagedAttentionArgs& p, const Workspace& ws, hipStream_t s);
// Copies positions [0, length) of batch index `index` of a contiguous cache
// [batch, layers, 2, max_seq, kv_heads, head_dim] into the pages `table`
// (pages_per_seq ids) of a pool [layers][num_pages][2][page_size][row_floats]
// with row_floats = kv_heads * head_dim (a multiple of 4). The caller checks
// the table.
hipError_t launch_paged_store(const float* state, float* pool, const uint32_t* table, uint64_t index,
                              uint64_t layers, uint64_t max_seq, uint64_t row_floats, uint64_t num_pages,
                              uint64_t page_size, uint64_t length, hipStream_t s);
uint64_t paged_attention_workspace_floats(const PagedAttentionArgs& p);

// ---- dense f32 matmul (reference/matmul.rs) ----
// out[b] = a[b or 0] x op(b[b or 0]); op = transpose when `nt`.
hipError_t launch_matmul(const float* a, const float* b, float* out, uint64_t batch, uint64_t batch_a,
                         uint64_t batch_b, uint64_t m, uint64_t k, uint64_t n, bool nt, hipStream_t s);

// ---- group-quantized weights (device-private layouts, see qmatmul.hip) ----
enum class QuantLayout : uint32_t {
    RowMajor = 0,  // payload bytes with offset-binary codes
    Mfma = 1,      // 16-row x 128-k superblocks in MFMA operand order
};
struct QuantWeight {
    const uint8_t* tiles;  // device-private copy of the codes
    const float* scales;   // [n, k / group]
    uint32_t format;       // sl_qformat
    uint32_t group;
    uint64_t n, k;
    QuantLayout layout;
    const float* tile_scales;  // Mfma: scales in wave order (quant_tile_scale_floats), else null
};
QuantLayout quant_layout_for(uint32_t format, uint64_t n, uint64_t k, uint32_t group);
uint64_t quant_tile_bytes(uint32_t format, uint64_t n, uint64_t k, QuantLayout layout);
// Builds the private copy from the row-major payload.
hipError_t launch_quant_repack(const uint8_t* payload, uint8_t* tiles, uint32_t format, uint64_t n,
                               uint64_t k, QuantLayout layout, hipStream_t s);
// Scales in wave order for the Mfma layout: [ceil(n/16)][k/128][16][gps]
// with gps = 2 for group 64 (both groups of a superblock), else 1 (the group
// containing the superblock); rows past n zero.
uint64_t quant_tile_scale_floats(uint64_t n, uint64_t k, uint32_t group, QuantLayout layout);
hipError_t launch_scale_repack(const float* scales, float* tile_scales, uint64_t n, uint64_t k, uint32_t group,
                               hipStream_t s);
// out[m, n] = sum_k a[m, k] * dequant(w)[n, k]  (a: [m, k] row-major)
// m > 16 on the Mfma layout (k % 128 == 0): fp16 matrix cores on activations
// split into two fp16 parts per element; hipErrorNotSupported when the
// shape or the workspace does not fit (nothing launched).
hipError_t launch_qgemm_mfma(const float* a, const QuantWeight& w, float* out, uint64_t m, const Workspace& ws,
                             hipStream_t s);
// The same for up to three weights of equal k, group and format that read
// the same activations (one activation split, one launch): out[i] =
// a * dequant(w[i])^T. With u, the activations are silu(a) * u (SwiGlu's
// down projection, elementwise); with out2[i] set, also out2[i] = resid[i]
// + out[i] (a residual Add), and out[i] may then be null (the product
// itself not written, when nothing reads it). With gamma (and no u), the
// activations are RMSNorm(a) * gamma (epsilon eps), formed by the
// activation split bit-identical to launch_rms_norm's vectorised kernel (the
// normalised rows are not written anywhere); qgemm_norm_takes says whether
// k and gamma allow it. qgemm_mfma_takes says whether a launch would run.
bool qgemm_mfma_takes(const float* a, const QuantWeight* const* w, uint32_t nseg, uint64_t m, const Workspace& ws);
bool qgemm_norm_takes(uint64_t k, const float* gamma);
hipError_t launch_qgemm_multi(const float* a, const QuantWeight* const* w, float* const* out, uint32_t nseg,
                              uint64_t m, const Workspace& ws, hipStream_t s, const float* u = nullptr,
                              const float* const* resid = nullptr, float* const* out2 = nullptr,
                              const float* gamma = nullptr, float eps = 0.f);
hipError_t launch_qmatmul(const float* a, const QuantWeight& w, float* out, uint64_t m, const Workspace& ws,
                          hipStream_t s);
// The MFMA decode path (m <= 16, Mfma layout); returns hipErrorNotSupported
// for shapes it does not take.
hipError_t launch_qgemv_mfma(const float* a, const QuantWeight& w, float* out, uint64_t m, const Workspace& ws,
                             hipStream_t s);

// ---- composites ----
// Decode GEMV with the K reduction inside one workgroup and its fusions
// (qgemv_fused.hip). Needs QuantLayout::Mfma weights of one format, group
// and k, m <= 16, m * k <= 16384, k % 256 == 0, group 64/128/256 or a
// multiple of 256, 16-byte aligned a / gamma / normed; otherwise returns
// hipErrorNotSupported before launching anything.
constexpr uint32_t kFusedMaxSegs = 3;
constexpr uint32_t kFusedPlain = 0;     // out[i] = a x w[i]^T
constexpr uint32_t kFusedResidual = 1;  // ... and out2[i] = resid[i] + out[i]
constexpr uint32_t kFusedPair = 2;      // out[0] = silu(a x w[0]^T) * (a x w[1]^T)
struct QgemvFused {
    const float* a;       // [m, k]
    const float* gamma;   // RMSNorm weight [k] applied to a first, or null
    float* normed;        // where the normalised a is written (gamma set), or null
    float eps;
    const QuantWeight* w[kFusedMaxSegs];
    float* out[kFusedMaxSegs];
    const float* resid[kFusedMaxSegs];
    float* out2[kFusedMaxSegs];
    uint32_t nseg;
    uint64_t m;
    uint32_t epilogue;
    // scratch for the k-slice partial sums of a single weight whose m x k
    // activations exceed the kernel's LDS (the down projection at batch 8),
    // or null: such a shape is then not taken
    float* partial = nullptr;
    uint64_t partial_floats = 0;
};
hipError_t launch_qgemv_fused(const QgemvFused& f, hipStream_t s);

// Weights are dense f32 (pointer) or quantized (QuantWeight with tiles != null).
struct WeightRef {
    const float* dense;
    QuantWeight quant;
    bool quantized() const { return quant.tiles != nullptr; }
};
hipError_t launch_linear(const float* a, const WeightRef& w, float* out, uint64_t rows, uint64_t n,
                         uint64_t k, const Workspace& ws, hipStream_t s);
// Rows per chunk of launch_swiglu for a workspace of ws_floats floats.
uint64_t swiglu_chunk_rows(uint64_t ws_floats, uint64_t inter);
// SwiGlu (reference/swiglu.rs): out = (silu(x Wg^T) * (x Wu^T)) Wd^T.
// With out2, also out2 = resid + out (a residual Add after the SwiGlu);
// out_dead: nothing reads out afterwards, so the q-GEMM route may skip it.
// With gamma, x is normalised first (RMSNorm, epsilon eps) inside the gate/up
// q-GEMM's activation split; hipErrorNotSupported, before anything is
// launched, unless every row chunk takes that route.
hipError_t launch_swiglu(const float* x, const WeightRef& gate, const WeightRef& up,
                         const WeightRef& down, float* out, uint64_t rows, uint64_t hidden,
                         uint64_t inter, const Workspace& ws, hipStream_t s, const float* resid = nullptr,
                         float* out2 = nullptr, bool out_dead = false, const float* gamma = nullptr,
                         float eps = 0.f);
// gate/up epilogue: h = silu(g) * u, elementwise over n values.
hipError_t launch_silu_mul(const float* g, const float* u, float* h, uint64_t n, hipStream_t s);
// RmsNormMatMul (reference/fused.rs): out = rms_norm(x, weight) W^T.
hipError_t launch_rms_norm_matmul(const float* x, const float* weight, const WeightRef& w, float* out,
                                  uint64_t rows, uint64_t hidden, uint64_t out_features, float eps,
                                  const Workspace& ws, hipStream_t s);

}  // namespace slhip
