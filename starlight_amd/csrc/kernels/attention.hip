// CausalAttention (reference/attention.rs:129-219) after its kv_append.
//
// For query (b, h, t) the visible keys are 0..=past_len+t of KV head
// h / (heads / kv_heads), read from cache[b, layer, 0/1, j, kv_head, :]
// (attention.rs:8-31). The reference scans the keys three times
// (max, denominator, weighted sum); here every key is read once with a running
// maximum (online softmax): m' = max(m, s), l' = l*e^(m-m') + e^(s-m'),
// acc' = acc*e^(m-m') + e^(s-m')*v, out = acc / l. Same mathematics, one pass.
//
// Kernels:
//  * attn_decode + attn_decode_merge — decode and short chunks (group * seq
//    <= 16 query rows per KV head). A block owns one (batch, KV head, 32-key
//    chunk); all query rows sharing that KV head are served from one read of
//    the chunk's K/V rows through LDS. Rows at or after past_len come from the
//    new K/V and the owning block appends them to the cache (kv_append fused).
//    The grid depends only on max_seq; chunks past the current length exit.
//    Partial (m, l, acc) go to the workspace and the merge kernel combines the
//    active chunks in order.
//  * attn_split / attn_merge — other decode shapes: one wave per
//    (b, h, t, key chunk), score by wave reduction, then a merge kernel.
//  * attn_tiled — prefill: a block owns 64 queries of one head, two threads
//    per query (each half of head_dim), and streams 32-key K/V tiles through
//    LDS, so each K/V row read from L2 serves 64 queries.
#include "common.h"
#include "kernels.h"

namespace slhip {
namespace {

struct Geo {
    const float* q;
    const float* k_new;
    const float* v_new;
    float* wcache;
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


constexpr int kDecodeRows = 16;  // query rows (group * seq) per KV head

// One block per (key chunk of KT keys, KV head, batch); chunks at or beyond
// past_len + seq exit at once, so the grid (fixed by max_seq) can be replayed
// for any length. LDS: q [R][D], k/v [KT][D + 1], p [R][KT]. Every global
// load of a stage is issued before any is used.
template <int KT, bool VEC>
__global__ __launch_bounds__(256) void attn_decode(Geo g) {
    extern __shared__ float lds[];
    __shared__ float m_row[kDecodeRows], l_row[kDecodeRows];
    const uint32_t D = g.head_dim, S = g.seq, G = g.group;
    const uint32_t R = G * S;  // query rows: r = gi * S + t
    const uint32_t c = blockIdx.x, kvh = blockIdx.y;
    const uint64_t b = blockIdx.z;
    const int tid = threadIdx.x;
    const uint32_t keys = g.past_len + S;
    const uint32_t j0 = c * KT;
    if (j0 >= keys) return;
    const uint32_t nk = min(static_cast<uint32_t>(KT), keys - j0);
    float* qs = lds;                 // [R][D]
    float* ks = qs + R * D;          // [KT][D + 1]
    float* vs = ks + KT * (D + 1);   // [KT][D + 1]
    float* ps = vs + KT * (D + 1);   // [R][KT]
    const uint64_t time_stride = static_cast<uint64_t>(g.kv_heads) * D;
    float* kbase = g.wcache + b * g.batch_stride + g.layer_offset + kvh * D;
    float* vbase = kbase + g.parity_stride;

    if constexpr (VEC) {
        const uint32_t d4 = D / 4;
        // q rows of this KV head's query group
        constexpr int kQ = kDecodeRows * 256 / 4 / 256;  // float4 per thread, worst case
        float4 qv[kQ];
#pragma unroll
        for (int u = 0; u < kQ; ++u) {
            const uint32_t i = tid + 256 * u;
            qv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < R * d4) {
                const uint32_t r = i / d4, dd = i % d4, gi = r / S, t = r % S;
                qv[u] = reinterpret_cast<const float4*>(g.q + ((b * g.heads + kvh * G + gi) * S + t) * D)[dd];
            }
        }
        // K/V rows: cached rows from the cache, new rows from k_new/v_new
        constexpr int kKV = KT * 256 / 4 / 256;  // float4 per thread, worst case (D <= 256)
        float4 kv[kKV], vv[kKV];
#pragma unroll
        for (int u = 0; u < kKV; ++u) {
            const uint32_t i = tid + 256 * u;
            kv[u] = vv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < KT * d4) {
                const uint32_t jj = i / d4, dd = i % d4, j = j0 + jj;
                if (jj < nk) {
                    if (j < g.past_len) {
                        kv[u] = reinterpret_cast<const float4*>(kbase + j * time_stride)[dd];
                        vv[u] = reinterpret_cast<const float4*>(vbase + j * time_stride)[dd];
                    } else {
                        const uint64_t src = ((b * g.kv_heads + kvh) * S + (j - g.past_len)) * D;
                        kv[u] = reinterpret_cast<const float4*>(g.k_new + src)[dd];
                        vv[u] = reinterpret_cast<const float4*>(g.v_new + src)[dd];
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kQ; ++u) {
            const uint32_t i = tid + 256 * u;
            if (i < R * d4) reinterpret_cast<float4*>(qs)[i] = qv[u];
        }
#pragma unroll
        for (int u = 0; u < kKV; ++u) {
            const uint32_t i = tid + 256 * u;
            if (i < KT * d4) {
                const uint32_t jj = i / d4, d = 4 * (i % d4), j = j0 + jj;
                float* kr = ks + jj * (D + 1) + d;
                float* vr = vs + jj * (D + 1) + d;
                kr[0] = kv[u].x; kr[1] = kv[u].y; kr[2] = kv[u].z; kr[3] = kv[u].w;
                vr[0] = vv[u].x; vr[1] = vv[u].y; vr[2] = vv[u].z; vr[3] = vv[u].w;
                if (jj < nk && j >= g.past_len) {  // kv_append of the new rows
                    reinterpret_cast<float4*>(kbase + j * time_stride)[i % d4] = kv[u];
                    reinterpret_cast<float4*>(vbase + j * time_stride)[i % d4] = vv[u];
                }
            }
        }
    } else {
        for (uint32_t i = tid; i < R * D; i += 256) {
            const uint32_t r = i / D, d = i % D, gi = r / S, t = r % S;
            qs[i] = g.q[((b * g.heads + kvh * G + gi) * S + t) * D + d];
        }
        for (uint32_t i = tid; i < KT * D; i += 256) {
            const uint32_t jj = i / D, d = i % D, j = j0 + jj;
            float kx = 0.f, vx = 0.f;
            if (jj < nk) {
                if (j < g.past_len) {
                    kx = kbase[j * time_stride + d];
                    vx = vbase[j * time_stride + d];
                } else {
                    const uint64_t src = ((b * g.kv_heads + kvh) * S + (j - g.past_len)) * D + d;
                    kx = g.k_new[src];
                    vx = g.v_new[src];
                    kbase[j * time_stride + d] = kx;
                    vbase[j * time_stride + d] = vx;
                }
            }
            ks[jj * (D + 1) + d] = kx;
            vs[jj * (D + 1) + d] = vx;
        }
    }
    __syncthreads();
    // scores: one (row, key) pair per thread
    for (uint32_t i = tid; i < R * KT; i += 256) {
        const uint32_t r = i / KT, jj = i % KT;
        const float* qr = qs + r * D;
        const float* kr = ks + jj * (D + 1);
        float dot = 0.f;
        for (uint32_t d = 0; d < D; ++d) dot = fmaf(qr[d], kr[d], dot);
        const bool vis = jj < nk && j0 + jj <= g.past_len + r % S;
        ps[i] = vis ? dot * g.scale : -INFINITY;
    }
    __syncthreads();
    // chunk softmax per row: m = max, p = exp(s - m), l = sum p
    if (tid < static_cast<int>(R)) {
        float* pr = ps + tid * KT;
        float mx = -INFINITY;
        for (int jj = 0; jj < KT; ++jj) mx = fmaxf(mx, pr[jj]);
        float sum = 0.f;
        for (int jj = 0; jj < KT; ++jj) {
            const float e = mx == -INFINITY ? 0.f : expf(pr[jj] - mx);
            pr[jj] = e;
            sum += e;
        }
        m_row[tid] = mx;
        l_row[tid] = sum;
    }
    __syncthreads();
    // partial of this chunk: [(b, kvh)][chunk][r][2 + D]
    const uint64_t row_stride = 2 + D;
    float* part = g.ws + ((b * g.kv_heads + kvh) * g.chunks + c) * R * row_stride;
    for (uint32_t e = tid; e < R * D; e += 256) {
        const uint32_t r = e / D, d = e % D;
        const float* pr = ps + r * KT;
        float a = 0.f;
        for (int jj = 0; jj < KT; ++jj) a = fmaf(pr[jj], vs[jj * (D + 1) + d], a);
        part[r * row_stride + 2 + d] = a;
    }
    if (tid < static_cast<int>(R)) {
        part[tid * row_stride] = m_row[tid];
        part[tid * row_stride + 1] = l_row[tid];
    }
}

// Merges the chunk partials of one (batch, KV head): grid (kv_heads, batch).
__global__ __launch_bounds__(256) void attn_decode_merge(Geo g, uint32_t kt) {
    __shared__ float m_row[kDecodeRows], inv_row[kDecodeRows];
    const uint32_t D = g.head_dim, S = g.seq, G = g.group, R = G * S;
    const uint32_t kvh = blockIdx.x;
    const uint64_t b = blockIdx.y;
    const uint32_t active = (g.past_len + S + kt - 1) / kt;
    const uint64_t row_stride = 2 + D;
    const float* base = g.ws + (b * g.kv_heads + kvh) * g.chunks * R * row_stride;
    const int tid = threadIdx.x;
    if (tid < static_cast<int>(R)) {
        float mx = -INFINITY;
        for (uint32_t c = 0; c < active; ++c) mx = fmaxf(mx, base[(c * R + tid) * row_stride]);
        float l = 0.f;
        for (uint32_t c = 0; c < active; ++c) {
            const float* pc = base + (c * R + tid) * row_stride;
            if (pc[1] > 0.f) l += pc[1] * expf(pc[0] - mx);
        }
        m_row[tid] = mx;
        inv_row[tid] = 1.0f / l;
    }
    __syncthreads();
    for (uint32_t e = tid; e < R * D; e += 256) {
        const uint32_t r = e / D, d = e % D, gi = r / S, t = r % S;
        float a = 0.f;
        for (uint32_t c = 0; c < active; ++c) {
            const float* pc = base + (c * R + r) * row_stride;
            if (pc[1] > 0.f) a = fmaf(pc[2 + d], expf(pc[0] - m_row[r]), a);
        }
        g.out[((b * g.heads + kvh * G + gi) * S + t) * D + d] = a * inv_row[r];
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

hipError_t launch_attention(const AttentionArgs& a, const Workspace& ws, hipStream_t s) {
    const uint64_t queries = a.batch * a.heads * a.seq;
    if (queries == 0 || a.head_dim == 0) return hipSuccess;
    Geo g;
    g.q = a.q;
    g.k_new = a.k_new;
    g.v_new = a.v_new;
    g.wcache = a.cache;
    g.cache = a.cache;
    g.out = a.out;
    g.ws = ws.data;
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

    // Decode path: kv_append fused into the chunk kernel, then the merge.
    const uint64_t rows = static_cast<uint64_t>(g.group) * a.seq;
    const uint32_t kt = a.head_dim <= 128 ? 32 : 16;
    const uint64_t n_chunks = (a.max_seq + kt - 1) / kt;
    if (rows <= kDecodeRows && a.head_dim <= 256 && n_chunks <= 0xffffffffull &&
        a.batch * a.kv_heads * n_chunks * rows * (a.head_dim + 2) <= ws.floats) {
        g.chunks = static_cast<uint32_t>(n_chunks);
        g.chunk = kt;
        const bool vec = a.head_dim % 4 == 0 && aligned16(a.q) && aligned16(a.k_new) && aligned16(a.v_new) &&
                         aligned16(a.cache);
        dim3 grid(static_cast<unsigned>(n_chunks), g.kv_heads, static_cast<unsigned>(a.batch));
        const size_t lds = (rows * a.head_dim + 2 * kt * (a.head_dim + 1) + rows * kt) * sizeof(float);
        if (kt == 32) {
            if (vec) attn_decode<32, true><<<grid, 256, lds, s>>>(g);
            else attn_decode<32, false><<<grid, 256, lds, s>>>(g);
        } else {
            if (vec) attn_decode<16, true><<<grid, 256, lds, s>>>(g);
            else attn_decode<16, false><<<grid, 256, lds, s>>>(g);
        }
        attn_decode_merge<<<dim3(g.kv_heads, static_cast<unsigned>(a.batch)), 256, 0, s>>>(g, kt);
        return hipGetLastError();
    }

    hipError_t e = launch_kv_append(a.k_new, a.v_new, a.cache, a.batch, a.layers, a.layer, a.kv_heads, a.head_dim,
                                    a.max_seq, a.past_len, a.seq, s);
    if (e != hipSuccess) return e;
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
        const uint64_t by_ws = ws.floats / (queries * (a.head_dim + 2));
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
