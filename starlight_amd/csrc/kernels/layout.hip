// Data movement: Gather, LastToken, SplitHeads/MergeHeads
// (reference/layout.rs:25-166) and KvAppend (reference/attention.rs:33-83).
//
// All of them copy whole rows; a row is moved with 16-byte vectors when the
// row length and both base pointers allow it. Gather ids were range-checked on
// the host before the launch, as the reference checks every id before its
// first write (layout.rs:207-213).
#include "common.h"
#include "kernels.h"

namespace slhip {
namespace {

// One row of n > 0 elements (T = float4 or float) copied by a 256-thread
// block, U elements per thread and pass: each pass issues all of its loads
// before its first store, so a row of up to 256 U elements costs one memory
// round trip, not U of them. Loads and stores are unconditional (a guarded
// store pulls its load into the guard, and a load under a branch is waited
// for at the join): indices past the row re-read its last element and store
// it again, unchanged. The launcher picks U = ceil(n / 256) up to 4, so a
// row of up to 1024 elements has at most 255 such slots; a longer row's last
// pass has up to 1023.
template <int U, typename T>
__device__ __forceinline__ void copy_row(const T* __restrict__ src, T* __restrict__ dst, uint64_t n) {
    for (uint64_t c0 = threadIdx.x; c0 < n; c0 += U * 256) {
        T v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = src[min(c0 + u * 256, n - 1)];
#pragma unroll
        for (int u = 0; u < U; ++u) dst[min(c0 + u * 256, n - 1)] = v[u];
    }
}

// Gather: dst row r <- table row ids[r].
template <int U>
__global__ __launch_bounds__(256) void gather_rows(const float* __restrict__ table, const uint32_t* __restrict__ ids,
                                                   float* __restrict__ out, uint64_t hidden, bool vec) {
    const uint64_t r = blockIdx.x;
    const uint64_t src = static_cast<uint64_t>(ids[r]) * hidden;
    const uint64_t dst = r * hidden;
    if (vec)
        copy_row<U>(reinterpret_cast<const float4*>(table + src), reinterpret_cast<float4*>(out + dst), hidden / 4);
    else
        copy_row<U>(table + src, out + dst, hidden);
}

template <int U>
__global__ __launch_bounds__(256) void last_token_rows(const float* __restrict__ in, float* __restrict__ out,
                                                       uint64_t seq, uint64_t hidden, uint64_t position, bool vec) {
    const uint64_t b = blockIdx.x;
    const float* src = in + (b * seq + position) * hidden;
    float* dst = out + b * hidden;
    if (vec) copy_row<U>(reinterpret_cast<const float4*>(src), reinterpret_cast<float4*>(dst), hidden / 4);
    else copy_row<U>(src, dst, hidden);
}

// [B, S, H, D] <-> [B, H, S, D]: one thread per output element group of VEC.
template <int VEC, bool SPLIT>
__global__ __launch_bounds__(256) void heads_permute(const float* __restrict__ in, float* __restrict__ out,
                                                     uint64_t seq, uint64_t heads, uint64_t head_dim,
                                                     uint64_t total) {
    const uint64_t dv = head_dim / VEC;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        // i enumerates the output in its own layout.
        const uint64_t d = i % dv;
        uint64_t rest = i / dv;
        uint64_t b, h, t;
        if (SPLIT) {  // out [B, H, S, D]
            t = rest % seq; rest /= seq;
            h = rest % heads; b = rest / heads;
        } else {      // out [B, S, H, D]
            h = rest % heads; rest /= heads;
            t = rest % seq; b = rest / seq;
        }
        const uint64_t token_major = ((b * seq + t) * heads + h) * head_dim + d * VEC;
        const uint64_t head_major = ((b * heads + h) * seq + t) * head_dim + d * VEC;
        const uint64_t src = SPLIT ? token_major : head_major;
        const uint64_t dst = SPLIT ? head_major : token_major;
        if constexpr (VEC == 4)
            *reinterpret_cast<float4*>(out + dst) = *reinterpret_cast<const float4*>(in + src);
        else
            out[dst] = in[src];
    }
}

// k/v [B, Hkv, S, D] -> cache[b, layer, 0/1, past_len + t, h, :].
template <int VEC>
__global__ __launch_bounds__(256) void kv_append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                        float* __restrict__ cache, uint64_t kv_heads,
                                                        uint64_t head_dim, uint64_t seq, uint64_t batch_stride,
                                                        uint64_t layer_offset, uint64_t parity_stride,
                                                        uint64_t past_len, const uint32_t* __restrict__ dyn,
                                                        uint64_t total) {
    prefetch_kernarg<arg_bytes<const float*, const float*, float*, uint64_t, uint64_t, uint64_t, uint64_t, uint64_t, uint64_t, uint64_t, const uint32_t*, uint64_t>()>();
    if (dyn != nullptr) past_len = dyn[0];
    const uint64_t dv = head_dim / VEC;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        const uint64_t d = i % dv;
        uint64_t rest = i / dv;
        const uint64_t t = rest % seq; rest /= seq;
        const uint64_t h = rest % kv_heads;
        const uint64_t b = rest / kv_heads;
        const uint64_t src = ((b * kv_heads + h) * seq + t) * head_dim + d * VEC;
        const uint64_t dst = b * batch_stride + layer_offset + (past_len + t) * kv_heads * head_dim +
                             h * head_dim + d * VEC;
        if constexpr (VEC == 4) {
            *reinterpret_cast<float4*>(cache + dst) = *reinterpret_cast<const float4*>(k + src);
            *reinterpret_cast<float4*>(cache + dst + parity_stride) = *reinterpret_cast<const float4*>(v + src);
        } else {
            cache[dst] = k[src];
            cache[dst + parity_stride] = v[src];
        }
    }
}

// Row `index` of a contiguous cache [B, layers, 2, max_seq, row] -> pages of
// a pool [layers][num_pages][2][page_size][row]: float4 i of every cached
// row of positions [0, length), position j in page table[j / page_size].
__global__ __launch_bounds__(256) void paged_store_rows(const float* __restrict__ state, float* __restrict__ pool,
                                                        const uint32_t* __restrict__ table, uint64_t index,
                                                        uint64_t layers, uint64_t max_seq, uint64_t row4,
                                                        uint64_t num_pages, uint64_t page_size, uint64_t length,
                                                        uint64_t total) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        const uint64_t c = i % row4;
        uint64_t rest = i / row4;
        const uint64_t j = rest % length;
        rest /= length;
        const uint64_t kv = rest % 2, layer = rest / 2;
        const uint64_t src = (((index * layers + layer) * 2 + kv) * max_seq + j) * row4 + c;
        const uint64_t dst = (((layer * num_pages + table[j / page_size]) * 2 + kv) * page_size + j % page_size) *
                                 row4 + c;
        reinterpret_cast<float4*>(pool)[dst] = reinterpret_cast<const float4*>(state)[src];
    }
}

}  // namespace

// elements per thread and pass of copy_row for a row of n elements
static int copy_per_thread(uint64_t n) { return n <= 256 ? 1 : n <= 512 ? 2 : n <= 768 ? 3 : 4; }

hipError_t launch_gather(const float* table, const uint32_t* ids, float* out, uint64_t rows,
                         uint64_t hidden, hipStream_t s) {
    if (rows == 0 || hidden == 0) return hipSuccess;
    const bool vec = hidden % 4 == 0 && aligned16(table) && aligned16(out);
    const dim3 grid(static_cast<unsigned>(rows));
    switch (copy_per_thread(vec ? hidden / 4 : hidden)) {
        case 1: gather_rows<1><<<grid, 256, 0, s>>>(table, ids, out, hidden, vec); break;
        case 2: gather_rows<2><<<grid, 256, 0, s>>>(table, ids, out, hidden, vec); break;
        case 3: gather_rows<3><<<grid, 256, 0, s>>>(table, ids, out, hidden, vec); break;
        default: gather_rows<4><<<grid, 256, 0, s>>>(table, ids, out, hidden, vec); break;
    }
    return hipGetLastError();
}

hipError_t launch_last_token(const float* in, float* out, uint64_t batch, uint64_t seq, uint64_t hidden,
                             uint64_t seq_len, hipStream_t s) {
    if (batch == 0 || hidden == 0) return hipSuccess;
    const bool vec = hidden % 4 == 0 && aligned16(in) && aligned16(out);
    const dim3 grid(static_cast<unsigned>(batch));
    switch (copy_per_thread(vec ? hidden / 4 : hidden)) {
        case 1: last_token_rows<1><<<grid, 256, 0, s>>>(in, out, seq, hidden, seq_len - 1, vec); break;
        case 2: last_token_rows<2><<<grid, 256, 0, s>>>(in, out, seq, hidden, seq_len - 1, vec); break;
        case 3: last_token_rows<3><<<grid, 256, 0, s>>>(in, out, seq, hidden, seq_len - 1, vec); break;
        default: last_token_rows<4><<<grid, 256, 0, s>>>(in, out, seq, hidden, seq_len - 1, vec); break;
    }
    return hipGetLastError();
}

hipError_t launch_heads_permute(const float* in, float* out, uint64_t batch, uint64_t seq,
                                uint64_t heads, uint64_t head_dim, bool split, hipStream_t s) {
    const uint64_t elements = batch * seq * heads * head_dim;
    if (elements == 0) return hipSuccess;
    const bool vec = head_dim % 4 == 0 && aligned16(in) && aligned16(out);
    const uint64_t total = vec ? elements / 4 : elements;
    const unsigned grid = grid_for(total, 256, 256 * 8);
    if (vec) {
        if (split) heads_permute<4, true><<<grid, 256, 0, s>>>(in, out, seq, heads, head_dim, total);
        else heads_permute<4, false><<<grid, 256, 0, s>>>(in, out, seq, heads, head_dim, total);
    } else {
        if (split) heads_permute<1, true><<<grid, 256, 0, s>>>(in, out, seq, heads, head_dim, total);
        else heads_permute<1, false><<<grid, 256, 0, s>>>(in, out, seq, heads, head_dim, total);
    }
    return hipGetLastError();
}

hipError_t launch_kv_append(const float* k, const float* v, float* cache, uint64_t batch,
                            uint64_t layers, uint64_t layer, uint64_t kv_heads, uint64_t head_dim,
                            uint64_t max_seq, uint64_t past_len, uint64_t seq, const uint32_t* dyn,
                            hipStream_t s) {
    const uint64_t elements = batch * kv_heads * seq * head_dim;
    if (elements == 0) return hipSuccess;
    const uint64_t parity_stride = max_seq * kv_heads * head_dim;
    const uint64_t layer_stride = 2 * parity_stride;
    const uint64_t batch_stride = layers * layer_stride;
    const bool vec = head_dim % 4 == 0 && aligned16(k) && aligned16(v) && aligned16(cache);
    const uint64_t total = vec ? elements / 4 : elements;
    const unsigned grid = grid_for(total, 256, 256 * 8);
    if (vec)
        kv_append_kernel<4><<<grid, 256, 0, s>>>(k, v, cache, kv_heads, head_dim, seq, batch_stride,
                                                 layer * layer_stride, parity_stride, past_len, dyn, total);
    else
        kv_append_kernel<1><<<grid, 256, 0, s>>>(k, v, cache, kv_heads, head_dim, seq, batch_stride,
                                                 layer * layer_stride, parity_stride, past_len, dyn, total);
    return hipGetLastError();
}

hipError_t launch_paged_store(const float* state, float* pool, const uint32_t* table, uint64_t index,
                              uint64_t layers, uint64_t max_seq, uint64_t row_floats, uint64_t num_pages,
                              uint64_t page_size, uint64_t length, hipStream_t s) {
    if (row_floats % 4 != 0 || !aligned16(state) || !aligned16(pool) || page_size == 0) return hipErrorInvalidValue;
    const uint64_t row4 = row_floats / 4, total = layers * 2 * length * row4;
    if (total == 0) return hipSuccess;
    paged_store_rows<<<grid_for(total, 256, 256 * 16), 256, 0, s>>>(state, pool, table, index, layers, max_seq, row4,
                                                                   num_pages, page_size, length, total);
    return hipGetLastError();
}

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_layout() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&gather_rows<4>));
}

}  // namespace slhip
