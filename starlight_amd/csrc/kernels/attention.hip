// CausalAttention (reference/attention.rs:129-219) after its kv_append.
//
// For query (b, h, t) the visible keys are 0..=past_len+t of KV head
// h / (heads / kv_heads), read from cache[b, layer, 0/1, j, kv_head, :]
// (attention.rs:8-31). The reference scans the keys three times
// (max, denominator, weighted sum); here every key is read once with a running
// maximum (online softmax): m' = max(m, s), l' = l*e^(m-m') + e^(s-m'),
// acc' = acc*e^(m-m') + e^(s-m')*v, out = acc / l. Same mathematics, one pass.
//
// Two kernels:
//  * attn_split — one wave per (b, h, t, key chunk). Lanes split head_dim,
//    the score is a wave reduction. The chunk count is chosen so decode
//    (seq = 1) still launches thousands of waves (flash-decoding); partial
//    (m, l, acc) go to the workspace and attn_merge combines them. With one
//    chunk it writes the output directly.
//  * attn_tiled — prefill: a block owns 64 queries of one head, two threads
//    per query (each half of head_dim), and streams 32-key K/V tiles through
//    LDS, so each K/V row read from L2 serves 64 queries.
#include "common.h"
#include "kernels.h"

namespace slhip {
namespace {

struct Geo {
    const float* q;
    const float* cache;
    float* out;
    float* ws;
    uint32_t heads, kv_heads, seq, head_dim, group;
    uint32_t past_len, chunk, chunks;
    uint64_t batch_stride, layer_offset, parity_stride;  // elements
    float scale;
};

template <int DPL>  // head_dim <= 64 * DPL
__global__ __launch_bounds__(256) void attn_split(Geo g, uint64_t items) {
    const uint64_t item = static_cast<uint64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (item >= items) return;
    const int lane = threadIdx.x % kWave;
    // item = (((b*seq + t)*kv_heads + kvh)*chunks + c)*group + gi: the waves
    // sharing one KV chunk are neighbours.
    uint64_t rest = item;
    const uint32_t gi = rest % g.group; rest /= g.group;
    const uint32_t c = rest % g.chunks; rest /= g.chunks;
    const uint32_t kvh = rest % g.kv_heads; rest /= g.kv_heads;
    const uint32_t t = rest % g.seq;
    const uint64_t b = rest / g.seq;
    const uint32_t h = kvh * g.group + gi;
    const uint32_t key_count = g.past_len + t + 1;
    const uint32_t k0 = c * g.chunk;
    const uint32_t k1 = min(k0 + g.chunk, key_count);
    const uint64_t qrow = ((b * g.heads + h) * g.seq + t) * g.head_dim;

    float qv[DPL], acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
        const uint32_t d = lane + i * kWave;
        qv[i] = d < g.head_dim ? g.q[qrow + d] : 0.f;
        acc[i] = 0.f;
    }
    const uint64_t time_stride = static_cast<uint64_t>(g.kv_heads) * g.head_dim;
    const float* kbase = g.cache + b * g.batch_stride + g.layer_offset + kvh * g.head_dim;
    const float* vbase = kbase + g.parity_stride;
    float m = -INFINITY, l = 0.f;
    for (uint32_t j = k0; j < k1; ++j) {
        const float* kr = kbase + j * time_stride;
        const float* vr = vbase + j * time_stride;
        float part = 0.f, vv[DPL];
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
            const uint32_t d = lane + i * kWave;
            const bool in = d < g.head_dim;
            part = fmaf(qv[i], in ? kr[d] : 0.f, part);
            vv[i] = in ? vr[d] : 0.f;
        }
        const float s = wave_sum(part) * g.scale;
        const float m_new = fmaxf(m, s);
        const float corr = expf(m - m_new);
        const float p = expf(s - m_new);
        l = l * corr + p;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] = fmaf(acc[i], corr, p * vv[i]);
        m = m_new;
    }
    if (g.chunks == 1) {
        const float inv = 1.0f / l;
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
            const uint32_t d = lane + i * kWave;
            if (d < g.head_dim) g.out[qrow + d] = acc[i] * inv;
        }
        return;
    }
    // partial layout: [(b, h, t)][chunk][head_dim + 2]
    float* part = g.ws + (((b * g.heads + h) * g.seq + t) * g.chunks + c) * (g.head_dim + 2);
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
        const uint32_t d = lane + i * kWave;
        if (d < g.head_dim) part[2 + d] = acc[i];
    }
    if (lane == 0) {
        part[0] = m;
        part[1] = l;
    }
}

// Combines the chunk partials of one (b, h, t) per block.
__global__ __launch_bounds__(256) void attn_merge(Geo g) {
    const uint64_t bht = blockIdx.x;  // (b*heads + h)*seq + t
    const float* base = g.ws + bht * g.chunks * (g.head_dim + 2);
    float mx = -INFINITY;
    for (uint32_t c = 0; c < g.chunks; ++c) mx = fmaxf(mx, base[c * (g.head_dim + 2)]);
    float l = 0.f;
    for (uint32_t c = 0; c < g.chunks; ++c) {
        const float* p = base + c * (g.head_dim + 2);
        if (p[1] > 0.f) l += p[1] * expf(p[0] - mx);
    }
    const float inv = 1.0f / l;
    float* out = g.out + bht * g.head_dim;
    for (uint32_t d = threadIdx.x; d < g.head_dim; d += blockDim.x) {
        float a = 0.f;
        for (uint32_t c = 0; c < g.chunks; ++c) {
            const float* p = base + c * (g.head_dim + 2);
            if (p[1] > 0.f) a = fmaf(p[2 + d], expf(p[0] - mx), a);
        }
        out[d] = a * inv;
    }
}

constexpr int kTileQ = 64;  // queries per block
constexpr int kTileK = 32;  // keys per LDS tile

template <int D>
__global__ __launch_bounds__(128) void attn_tiled(Geo g) {
    constexpr int H = D / 2;  // dims per thread
    __shared__ float4 ks[kTileK * D / 4];
    __shared__ float4 vs[kTileK * D / 4];
    const uint32_t h = blockIdx.y;
    const uint64_t b = blockIdx.z;
    const uint32_t kvh = h / g.group;
    const int r = threadIdx.x / 2, half = threadIdx.x % 2;
    const uint32_t t = blockIdx.x * kTileQ + r;
    const bool valid = t < g.seq;
    const uint32_t key_count = g.past_len + t + 1;
    const uint32_t last_t = min(g.seq, (blockIdx.x + 1) * kTileQ) - 1;
    const uint32_t block_keys = g.past_len + last_t + 1;

    const uint64_t qrow = ((b * g.heads + h) * g.seq + (valid ? t : 0)) * D + half * H;
    float qv[H], acc[H];
#pragma unroll
    for (int i = 0; i < H; i += 4) {
        float4 v4 = *reinterpret_cast<const float4*>(g.q + qrow + i);
        qv[i] = v4.x; qv[i + 1] = v4.y; qv[i + 2] = v4.z; qv[i + 3] = v4.w;
        acc[i] = acc[i + 1] = acc[i + 2] = acc[i + 3] = 0.f;
    }
    const uint64_t time_stride = static_cast<uint64_t>(g.kv_heads) * D;
    const float* kbase = g.cache + b * g.batch_stride + g.layer_offset + kvh * D;
    const float* vbase = kbase + g.parity_stride;
    float m = -INFINITY, l = 0.f;

    for (uint32_t kt = 0; kt < block_keys; kt += kTileK) {
        __syncthreads();
        for (int e = threadIdx.x; e < kTileK * D / 4; e += 128) {
            const uint32_t row = e / (D / 4), col = e % (D / 4);
            const uint32_t j = kt + row;
            float4 kk = make_float4(0.f, 0.f, 0.f, 0.f), vv = kk;
            if (j < block_keys) {
                kk = reinterpret_cast<const float4*>(kbase + j * time_stride)[col];
                vv = reinterpret_cast<const float4*>(vbase + j * time_stride)[col];
            }
            ks[e] = kk;
            vs[e] = vv;
        }
        __syncthreads();
        float s[kTileK];
        float tile_max = -INFINITY;
#pragma unroll
        for (int jj = 0; jj < kTileK; ++jj) {
            const float4* kr = ks + jj * (D / 4) + half * (H / 4);
            float part = 0.f;
#pragma unroll
            for (int i = 0; i < H / 4; ++i) {
                const float4 k4 = kr[i];
                part = fmaf(qv[4 * i], k4.x, part);
                part = fmaf(qv[4 * i + 1], k4.y, part);
                part = fmaf(qv[4 * i + 2], k4.z, part);
                part = fmaf(qv[4 * i + 3], k4.w, part);
            }
            part += __shfl_xor(part, 1, kWave);
            const bool vis = kt + jj < key_count;
            s[jj] = vis ? part * g.scale : -INFINITY;
            tile_max = fmaxf(tile_max, s[jj]);
        }
        if (tile_max == -INFINITY) continue;  // every key of this tile is masked for this query
        const float m_new = fmaxf(m, tile_max);
        const float corr = expf(m - m_new);
        l *= corr;
#pragma unroll
        for (int i = 0; i < H; ++i) acc[i] *= corr;
#pragma unroll
        for (int jj = 0; jj < kTileK; ++jj) {
            const float p = expf(s[jj] - m_new);
            l += p;
            const float4* vr = vs + jj * (D / 4) + half * (H / 4);
#pragma unroll
            for (int i = 0; i < H / 4; ++i) {
                const float4 v4 = vr[i];
                acc[4 * i] = fmaf(p, v4.x, acc[4 * i]);
                acc[4 * i + 1] = fmaf(p, v4.y, acc[4 * i + 1]);
                acc[4 * i + 2] = fmaf(p, v4.z, acc[4 * i + 2]);
                acc[4 * i + 3] = fmaf(p, v4.w, acc[4 * i + 3]);
            }
        }
        m = m_new;
    }
    if (!valid) return;
    const float inv = 1.0f / l;
    float* orow = g.out + ((b * g.heads + h) * g.seq + t) * D + half * H;
#pragma unroll
    for (int i = 0; i < H; i += 4)
        *reinterpret_cast<float4*>(orow + i) =
            make_float4(acc[i] * inv, acc[i + 1] * inv, acc[i + 2] * inv, acc[i + 3] * inv);
}

}  // namespace

hipError_t launch_attention(const AttentionArgs& a, float* workspace, uint64_t workspace_floats,
                            hipStream_t s) {
    const uint64_t queries = a.batch * a.heads * a.seq;
    if (queries == 0 || a.head_dim == 0) return hipSuccess;
    Geo g;
    g.q = a.q;
    g.cache = a.cache;
    g.out = a.out;
    g.ws = workspace;
    g.heads = static_cast<uint32_t>(a.heads);
    g.kv_heads = static_cast<uint32_t>(a.kv_heads);
    g.seq = static_cast<uint32_t>(a.seq);
    g.head_dim = static_cast<uint32_t>(a.head_dim);
    g.group = static_cast<uint32_t>(a.heads / a.kv_heads);
    g.past_len = static_cast<uint32_t>(a.past_len);
    g.parity_stride = a.max_seq * a.kv_heads * a.head_dim;
    g.layer_offset = a.layer * 2 * g.parity_stride;
    g.batch_stride = a.layers * 2 * g.parity_stride;
    g.scale = a.scale;

    const bool aligned = aligned16(a.q) && aligned16(a.cache) && aligned16(a.out);
    if (a.seq >= 16 && aligned && (a.head_dim == 64 || a.head_dim == 128)) {
        dim3 grid(static_cast<unsigned>((a.seq + kTileQ - 1) / kTileQ), g.heads, static_cast<unsigned>(a.batch));
        if (a.head_dim == 64) attn_tiled<64><<<grid, 128, 0, s>>>(g);
        else attn_tiled<128><<<grid, 128, 0, s>>>(g);
        return hipGetLastError();
    }
    if (a.head_dim > 256) return hipErrorInvalidValue;

    // Split the longest key range so that about 2048 waves run, each chunk
    // holding at least 64 keys, within the workspace.
    const uint64_t max_keys = a.past_len + a.seq;
    uint64_t chunks = 1;
    if (queries < 2048) {
        chunks = (2048 + queries - 1) / queries;
        const uint64_t by_keys = (max_keys + 63) / 64;
        if (chunks > by_keys) chunks = by_keys;
        const uint64_t by_ws = workspace_floats / (queries * (a.head_dim + 2));
        if (chunks > by_ws) chunks = by_ws;
        if (chunks < 1) chunks = 1;
    }
    g.chunk = static_cast<uint32_t>((max_keys + chunks - 1) / chunks);
    g.chunks = static_cast<uint32_t>(chunks);
    const uint64_t items = queries * chunks;
    const unsigned blocks = static_cast<unsigned>((items + 3) / 4);
    const int dpl = static_cast<int>((a.head_dim + 63) / 64);
    switch (dpl) {
        case 1: attn_split<1><<<blocks, 256, 0, s>>>(g, items); break;
        case 2: attn_split<2><<<blocks, 256, 0, s>>>(g, items); break;
        case 3: attn_split<3><<<blocks, 256, 0, s>>>(g, items); break;
        default: attn_split<4><<<blocks, 256, 0, s>>>(g, items); break;
    }
    if (chunks > 1) attn_merge<<<static_cast<unsigned>(queries), 128, 0, s>>>(g);
    return hipGetLastError();
}

}  // namespace slhip
