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
//    <= 16 query rows per KV head, head_dim a multiple of 64 up to 256): a
//    (P, kv_heads, batch) grid with P fixed by max_seq, so one launch shape
//    serves every past_len. 16-key tiles are dealt round-robin to the blocks'
//    waves, all query rows sharing a KV head are served from one read of
//    each K/V row, rows at or after past_len come from the new K/V and are
//    appended to the cache by the lane group that reads them (kv_append
//    fused). One partial (m, l, acc) per block; the merge kernel combines P.
//  * attn_split / attn_merge — other decode shapes: one wave per
//    (b, h, t, key chunk), score by wave reduction, then a merge kernel.
//  * attn_prefill — prefill (16 or more queries, head_dim 64 or 128): a block
//    owns 64 queries of one head (two query tiles in turn) and streams 32-key
//    K/V tiles through LDS; both products run on the f32 matrix cores. In the
//    fused form prefill_prep first splits, rotates and appends (one block per
//    token) and attn_prefill writes MergeHeads' layout.
#include "common.h"
#include "kernels.h"
#include "starlight_hip.h"

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
    const uint32_t* dyn;  // when set, dyn[0] is past_len
    // fused form: rope inputs and the extra outputs (see AttentionArgs)
    const uint32_t* pos;
    double theta;
    uint32_t rope_variant;
    float* merged;
    float* mirror;
    float* q_split;  // fused form: intermediates a later command reads, or null
    float* k_split;
    float* v_split;
    float* q_rot;
    float* k_rot;
    const float* rope_tab;  // fused form: the sine / cosine table, or null
    // paged form (attn_decode<.., PAGED>): key j of row b is slot j % page_size
    // of page block_table[b * pages_per_seq + j / page_size]; a page holds
    // K then V, [2][page_size][kv_heads][head_dim], page_stride elements, and
    // the layer's pages start at wcache + layer_offset; row b has seq_past[b]
    // cached keys before this step
    const uint32_t* block_table;
    const uint32_t* seq_past;
    uint32_t page_size, pages_per_seq;
    uint64_t page_stride;
};

__device__ __forceinline__ uint32_t past_of(const Geo& g) { return g.dyn != nullptr ? g.dyn[0] : g.past_len; }

template <int DPL>  // head_dim <= 64 * DPL
__global__ __launch_bounds__(256) void attn_split(Geo g, uint64_t items) {
    prefetch_kernarg<arg_bytes<Geo, uint64_t>()>();
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
    const uint32_t key_count = past_of(g) + t + 1;
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
    prefetch_kernarg<arg_bytes<Geo>()>();
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


// ---- decode: flash-decoding over a grid fixed by max_seq ----
//
// Keys are cut into tiles of 16. Tile i belongs to block i % P, wave
// (i / P) % 4 of that block, so every block of the (P, kv_heads, batch) grid
// gets an equal share at any length and the grid never depends on past_len.
// Inside a wave, four groups of 16 lanes each take 4 consecutive keys of the
// tile; a lane holds DV float4 of every key row (dims li*4 + 64*u), so a
// group reads each K/V row as contiguous 256-byte runs and all 8*DV loads of
// a tile are in flight together. Scores are reduced across the 16 lanes of a
// group; each group keeps its own online-softmax state (m, l, acc) for the
// RT query rows of this KV head, the groups and then the waves are combined,
// and the block writes one partial [(b, kvh, p)][r][4 + D] = (m, l, -, -,
// acc). Rows j >= past_len come from k_new / v_new and the lane group that
// reads one also appends it to the cache.
constexpr int kDecodeLanes = 16;                       // lanes per key
constexpr int kDecodeKeys = 4;                         // keys per lane group per tile, at most
constexpr int kDecodeTile = kDecodeKeys * kWave / kDecodeLanes;  // 16 keys per wave tile, at most
constexpr int kDecodeMaxRows = 16;
constexpr uint32_t kDecodePartStride = 4;              // floats before acc in a partial row

__device__ __forceinline__ float group_sum16(float v) { return row_sum(v); }  // a lane group is a DPP row

__device__ __forceinline__ float4 f4_fma(float a, float4 x, float4 y) {
    return make_float4(fmaf(a, x.x, y.x), fmaf(a, x.y, y.y), fmaf(a, x.z, y.z), fmaf(a, x.w, y.w));
}

__device__ __forceinline__ float4 f4_scale(float4 x, float a) { return make_float4(x.x * a, x.y * a, x.z * a, x.w * a); }

__device__ __forceinline__ void put4(float* p, float4 v) {
    p[0] = v.x;
    p[1] = v.y;
    p[2] = v.z;
    p[3] = v.w;
}

// Folds state (mo, lo, ao) into (m, l, a); an empty state has m == -inf.
template <int DV>
__device__ __forceinline__ void fold_state(float& m, float& l, float4 (&a)[DV], float mo, float lo,
                                           const float4 (&ao)[DV]) {
    const float mn = fmaxf(m, mo);
    if (mn == -INFINITY) return;
    const float ca = m == -INFINITY ? 0.f : expf(m - mn);
    const float cb = mo == -INFINITY ? 0.f : expf(mo - mn);
    l = l * ca + lo * cb;
#pragma unroll
    for (int u = 0; u < DV; ++u) a[u] = f4_fma(cb, ao[u], f4_scale(a[u], ca));
    m = mn;
}

// Rope rotation of one pair, as reference/rope.rs (and rope.hip) computes it.
__device__ __forceinline__ void rotate(float& x, float& y, float sine, float cosine) {
    const float a = x * cosine - y * sine;
    const float b = x * sine + y * cosine;
    x = a;
    y = b;
}

// The pair angles' sine and cosine for token t: sc[t * D + pair] = sin,
// sc[t * D + D/2 + pair] = cos, from f64 pow / sin / cos rounded once.
__device__ __forceinline__ void rope_table(const Geo& g, uint64_t b, uint32_t S, uint32_t D, float* sc) {
    const uint32_t half = D / 2;
    for (uint32_t i = threadIdx.x; i < S * half; i += blockDim.x) {
        const uint32_t t = i / half, pair = i % half;
        const double position = static_cast<double>(g.pos[b * S + t]);
        const double angle = position / pow(g.theta, 2.0 * static_cast<double>(pair) / static_cast<double>(D));
        sc[t * D + pair] = static_cast<float>(sin(angle));
        sc[t * D + half + pair] = static_cast<float>(cos(angle));
    }
}

__global__ __launch_bounds__(256) void rope_sincos(const uint32_t* __restrict__ pos, uint32_t tokens, uint32_t D,
                                                   double theta, float* __restrict__ table) {
    const uint32_t half = D / 2;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= tokens * half) return;
    const uint32_t t = i / half, pair = i % half;
    const double position = static_cast<double>(pos[t]);
    const double angle = position / pow(theta, 2.0 * static_cast<double>(pair) / static_cast<double>(D));
    table[t * D + pair] = static_cast<float>(sin(angle));
    table[t * D + half + pair] = static_cast<float>(cos(angle));
}

// KEYS: keys per lane group per tile (a wave tile is 4 KEYS keys). Each
// wave streams whole tiles, so a wave holding one tile more than the others
// sets the launch's length: where the grid has few waves per key range
// (batch > 1, partials capped by the grid size) 8-key tiles even that out,
// and where every wave holds one tile or none (batch 1) 16-key tiles are
// cheaper. The leading arguments (preloaded into scalar registers with the wave)
// are what the first loads need: past_len's source (dyn, seq_past for the
// paged form, or null for past_fixed), the query rows and their geometry
// (seq, group, heads). The past_len and query loads go out at once, and the
// argument block is fetched meanwhile.
template <int DV, int RT, bool FUSED, bool PAGED, int KEYS>
__global__ __launch_bounds__(256) void attn_decode(const uint32_t* past_src, uint32_t past_fixed,
                                                   const float* q_in, uint32_t seq, uint32_t group, uint32_t heads,
                                                   Geo g) {
    constexpr int D4 = 16 * DV;  // float4 per row
    constexpr int kTileKeys = KEYS * kWave / kDecodeLanes;  // keys per wave tile
    extern __shared__ float sc[];  // FUSED: rope table [S][D]
    __shared__ float4 qs[RT * D4];
    // Softmax states combined through LDS at the end: with small per-lane
    // state (RT * DV <= 8) every lane group's own (16 per block: 32 KB for
    // head_dim 128, four rows), else one per wave after lane swaps.
    constexpr int NS = RT * DV <= 8 ? 16 : 4;
    __shared__ float4 wacc[NS][RT][D4];
    __shared__ float wml[NS][RT][2];
    const uint32_t S = seq, G = group, R = G * S;
    const uint32_t P = gridDim.x, p = blockIdx.x, kvh = blockIdx.y;
    const uint64_t b = blockIdx.z;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int grp = lane / kDecodeLanes, li = lane % kDecodeLanes;
    const uint32_t past = past_src != nullptr ? past_src[PAGED ? b : 0] : past_fixed, keys = past + S;
    const uint32_t ntiles = (keys + kTileKeys - 1) / kTileKeys;
    // query rows: loaded first (rows past R re-read row 0 and are zeroed),
    // staged in LDS after the first tile's loads have gone out
    constexpr int QPT = (RT * D4 + 255) / 256;
    float4 qv[QPT];
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const uint32_t i = min(static_cast<uint32_t>(tid + 256 * u), static_cast<uint32_t>(RT * D4 - 1));
        const uint32_t r = min(i / D4, R - 1), c = i % D4, gi = r / S, t = r % S;
        const uint64_t h = kvh * G + gi;
        const uint64_t row = FUSED ? (b * S + t) * heads + h : (b * heads + h) * S + t;
        qv[u] = reinterpret_cast<const float4*>(q_in + row * (4 * D4))[c];
    }
    // the rest of the arguments, in one batch of loads
    prefetch_kernarg<arg_bytes<const uint32_t*, uint32_t, const float*, uint32_t, uint32_t, uint32_t, Geo>()>();

    const uint64_t time_stride = static_cast<uint64_t>(g.kv_heads) * (4 * D4);
    float* kbase = g.wcache + (PAGED ? 0 : b * g.batch_stride) + g.layer_offset + kvh * (4 * D4);
    // K row j of this KV head (V is parity_stride further): contiguous, or
    // through the row's block table
    auto krow = [&](uint32_t j) -> float* {
        if constexpr (PAGED) {
            const uint32_t page = g.block_table[b * g.pages_per_seq + j / g.page_size];
            return kbase + page * g.page_stride + static_cast<uint64_t>(j % g.page_size) * time_stride;
        } else {
            return kbase + static_cast<uint64_t>(j) * time_stride;
        }
    };
    // K/V rows of a tile for this lane: cached rows from the cache, new rows
    // from k_new / v_new, zeros past the end.
    auto load_tile = [&](uint32_t tile, float4 (&kx)[KEYS][DV], float4 (&vx)[KEYS][DV]) {
        const uint32_t j0 = tile * kTileKeys + grp * KEYS;
#pragma unroll
        for (int kb = 0; kb < KEYS; ++kb) {
            // Every lane loads (keys past the end re-read the last row; their
            // scores are masked to -inf, so they weigh exactly 0), so the
            // loads carry no branch and the waits before their use are exact.
            const uint32_t j = min(j0 + kb, keys - 1);
            const float* kr = krow(j);
            const float* vr = kr + g.parity_stride;
            if (j >= past) {
                // [B, Hkv, S, D], or [B, S, Hkv * D] before SplitHeads (fused)
                const uint64_t t = j - past;
                const uint64_t src = (FUSED ? (b * S + t) * g.kv_heads + kvh : (b * g.kv_heads + kvh) * S + t) *
                                     (4 * D4);
                kr = g.k_new + src;
                vr = g.v_new + src;
            }
#pragma unroll
            for (int u = 0; u < DV; ++u) {
                kx[kb][u] = reinterpret_cast<const float4*>(kr)[li + 16 * u];
                vx[kb][u] = reinterpret_cast<const float4*>(vr)[li + 16 * u];
            }
        }
    };
    // The first tile's loads go out before the query rows are staged, and
    // each iteration starts the next tile's loads before computing.
    // FUSED: the first entries of the Rope table, loaded with the query rows
    // and ahead of the K/V tile, whose bytes they would otherwise wait behind
    // (every thread loads: without a table, from the query rows)
    constexpr int kTabRegs = 2;
    float tabv[kTabRegs];
    if constexpr (FUSED) {
        const uint32_t SD = S * 4 * D4;
        const float* tab = g.rope_tab != nullptr ? g.rope_tab + b * SD : q_in;
#pragma unroll
        for (int u = 0; u < kTabRegs; ++u) tabv[u] = tab[min(static_cast<uint32_t>(tid + 256 * u), SD - 1)];
    }
    uint32_t tile = p + P * wave;
    float4 kv[KEYS][DV], vv[KEYS][DV];
    // Every wave loads a first tile, unconditionally (a wave without one
    // re-reads the last key row, which its neighbours load too): loads
    // under a branch leave register copies at the join that wait for the
    // data right away, ahead of the query staging and Rope below.
    load_tile(tile, kv, vv);
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const uint32_t i = tid + 256 * u;
        if (i < RT * D4) qs[i] = i / D4 < R ? qv[u] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // the query rows of this KV head in SplitHeads layout [B, H, S, D]
    // (element stores: the buffers may sit at any offset)
    auto put_q_rows = [&](float* dst) {
        for (uint32_t i = tid; i < R * D4; i += 256) {
            const uint32_t r = i / D4, c = i % D4, t = r % S;
            const uint64_t h = kvh * G + r / S;
            put4(dst + ((b * g.heads + h) * S + t) * (4 * D4) + 4 * c, qs[i]);
        }
    };
    if constexpr (FUSED) {
        // Rope of the query rows, in LDS
        constexpr uint32_t D = 4 * D4;
        if (g.rope_tab != nullptr) {
#pragma unroll
            for (int u = 0; u < kTabRegs; ++u)
                if (tid + 256 * u < S * D) sc[tid + 256 * u] = tabv[u];
            for (uint32_t i = tid + 256 * kTabRegs; i < S * D; i += 256) sc[i] = g.rope_tab[b * S * D + i];
        } else {
            rope_table(g, b, S, D, sc);
        }
        __syncthreads();
        if (p == 0 && g.q_split != nullptr) {  // block-uniform
            put_q_rows(g.q_split);
            __syncthreads();  // the rotation below rewrites rows other threads store here
        }
        if (g.rope_variant == SL_ROPE_NEOX) {
            for (uint32_t i = tid; i < R * (D4 / 2); i += 256) {  // four pairs (d, d + D/2) per item
                const uint32_t r = i / (D4 / 2), c = i % (D4 / 2);
                const float* st = sc + (r % S) * D;
                float4 x = qs[r * D4 + c], y = qs[r * D4 + c + D4 / 2];
                rotate(x.x, y.x, st[4 * c], st[D / 2 + 4 * c]);
                rotate(x.y, y.y, st[4 * c + 1], st[D / 2 + 4 * c + 1]);
                rotate(x.z, y.z, st[4 * c + 2], st[D / 2 + 4 * c + 2]);
                rotate(x.w, y.w, st[4 * c + 3], st[D / 2 + 4 * c + 3]);
                qs[r * D4 + c] = x;
                qs[r * D4 + c + D4 / 2] = y;
            }
        } else {
            for (uint32_t i = tid; i < R * D4; i += 256) {  // pairs (2i, 2i + 1), two per float4
                const uint32_t r = i / D4, c = i % D4;
                const float* st = sc + (r % S) * D;
                float4 x = qs[r * D4 + c];
                rotate(x.x, x.y, st[2 * c], st[D / 2 + 2 * c]);
                rotate(x.z, x.w, st[2 * c + 1], st[D / 2 + 2 * c + 1]);
                qs[r * D4 + c] = x;
            }
        }
        __syncthreads();
        if (p == 0 && g.q_rot != nullptr) put_q_rows(g.q_rot);
    }
    __syncthreads();

    float m[RT], l[RT];
    float4 acc[RT][DV];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.f;
#pragma unroll
        for (int u = 0; u < DV; ++u) acc[r][u] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    for (; tile < ntiles; tile += 4 * P) {
        const uint32_t j0 = tile * kTileKeys + grp * KEYS;
        float4 kn[KEYS][DV], vn[KEYS][DV];
        // the next tile's loads only when there is one: loads still in flight
        // at the loop's end would hold the combine below (their registers are
        // reused), and most decode waves have a single tile
        const bool more = tile + 4 * P < ntiles;
        if (more) load_tile(tile + 4 * P, kn, vn);
#pragma unroll
        for (int kb = 0; kb < KEYS; ++kb) {
            const uint32_t j = j0 + kb;
            if (j >= past && j < keys) {
                // the new row in SplitHeads / Rope layout [B, Hkv, S, D]
                const uint64_t split_row = ((b * g.kv_heads + kvh) * S + (j - past)) * (4 * D4);
                if (FUSED && g.k_split != nullptr) {
#pragma unroll
                    for (int u = 0; u < DV; ++u) put4(g.k_split + split_row + 4 * (li + 16 * u), kv[kb][u]);
                }
                if (FUSED && g.v_split != nullptr) {
#pragma unroll
                    for (int u = 0; u < DV; ++u) put4(g.v_split + split_row + 4 * (li + 16 * u), vv[kb][u]);
                }
                if constexpr (FUSED) {
                    // Rope of a new key row before it is used and appended
                    constexpr uint32_t D = 4 * D4;
                    const float* st = sc + (j - past) * D;
                    if (g.rope_variant == SL_ROPE_NEOX && DV == 1) {
                        // head_dim 64: the pair of dim d < 32 is d + 32, four
                        // float4 further, in lane li ^ 8 of the same 16-lane
                        // group (DPP row rotate by 8); each lane keeps its
                        // half of rotate()'s result
                        float4& me = kv[kb][0];
                        const float4 pa = make_float4(dpp_f<kDppRowRor8>(me.x), dpp_f<kDppRowRor8>(me.y),
                                                      dpp_f<kDppRowRor8>(me.z), dpp_f<kDppRowRor8>(me.w));
                        const bool first = li < 8;
                        const uint32_t pr = 4 * (li & 7);  // pair index of the lane's first dim
                        const float mine[4] = {me.x, me.y, me.z, me.w}, other[4] = {pa.x, pa.y, pa.z, pa.w};
                        float res[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float sine = st[pr + e], cosine = st[D / 2 + pr + e];
                            res[e] = first ? mine[e] * cosine - other[e] * sine : other[e] * sine + mine[e] * cosine;
                        }
                        me = make_float4(res[0], res[1], res[2], res[3]);
                    } else if (g.rope_variant == SL_ROPE_NEOX) {
#pragma unroll
                        for (int u = 0; u < DV / 2; ++u) {  // pairs (d, d + D/2) sit in one lane
                            const uint32_t d = 4 * li + 64 * u;
                            float4& x = kv[kb][u];
                            float4& y = kv[kb][u + DV / 2];
                            rotate(x.x, y.x, st[d], st[D / 2 + d]);
                            rotate(x.y, y.y, st[d + 1], st[D / 2 + d + 1]);
                            rotate(x.z, y.z, st[d + 2], st[D / 2 + d + 2]);
                            rotate(x.w, y.w, st[d + 3], st[D / 2 + d + 3]);
                        }
                    } else {
#pragma unroll
                        for (int u = 0; u < DV; ++u) {
                            const uint32_t pr = (4 * li + 64 * u) / 2;
                            float4& x = kv[kb][u];
                            rotate(x.x, x.y, st[pr], st[D / 2 + pr]);
                            rotate(x.z, x.w, st[pr + 1], st[D / 2 + pr + 1]);
                        }
                    }
                }
                if (FUSED && g.k_rot != nullptr) {
#pragma unroll
                    for (int u = 0; u < DV; ++u) put4(g.k_rot + split_row + 4 * (li + 16 * u), kv[kb][u]);
                }
#pragma unroll
                for (int u = 0; u < DV; ++u) {
                    float* const kw = krow(j);
                    reinterpret_cast<float4*>(kw)[li + 16 * u] = kv[kb][u];
                    reinterpret_cast<float4*>(kw + g.parity_stride)[li + 16 * u] = vv[kb][u];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            if (r >= static_cast<int>(R)) continue;
            float4 qv[DV];
#pragma unroll
            for (int u = 0; u < DV; ++u) qv[u] = qs[r * D4 + li + 16 * u];
            const uint32_t limit = past + r % S;  // last visible key of this row
            float s[KEYS];
            float tmax = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < KEYS; ++kb) {
                float dot = 0.f;
#pragma unroll
                for (int u = 0; u < DV; ++u) {
                    dot = fmaf(qv[u].x, kv[kb][u].x, dot);
                    dot = fmaf(qv[u].y, kv[kb][u].y, dot);
                    dot = fmaf(qv[u].z, kv[kb][u].z, dot);
                    dot = fmaf(qv[u].w, kv[kb][u].w, dot);
                }
                dot = group_sum16(dot);
                s[kb] = j0 + kb <= limit ? dot * g.scale : -INFINITY;
                tmax = fmaxf(tmax, s[kb]);
            }
            const float mn = fmaxf(m[r], tmax);
            if (mn == -INFINITY) continue;
            const float corr = m[r] == -INFINITY ? 0.f : expf(m[r] - mn);
            float lsum = l[r] * corr;
#pragma unroll
            for (int u = 0; u < DV; ++u) acc[r][u] = f4_scale(acc[r][u], corr);
#pragma unroll
            for (int kb = 0; kb < KEYS; ++kb) {
                const float pk = s[kb] == -INFINITY ? 0.f : expf(s[kb] - mn);
                lsum += pk;
#pragma unroll
                for (int u = 0; u < DV; ++u) acc[r][u] = f4_fma(pk, vv[kb][u], acc[r][u]);
            }
            l[r] = lsum;
            m[r] = mn;
        }
        if (more) {
#pragma unroll
            for (int kb = 0; kb < KEYS; ++kb) {
#pragma unroll
                for (int u = 0; u < DV; ++u) {
                    kv[kb][u] = kn[kb][u];
                    vv[kb][u] = vn[kb][u];
                }
            }
        }
    }

    // combine the lane groups and waves
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        if (r >= static_cast<int>(R)) continue;
        static_assert(kDecodeLanes == 16, "lane groups are 16-lane rows");
        if constexpr (NS == 16) {
            const int st = wave * 4 + grp;
#pragma unroll
            for (int u = 0; u < DV; ++u) wacc[st][r][li + 16 * u] = acc[r][u];
            if (li == 0) {
                wml[st][r][0] = m[r];
                wml[st][r][1] = l[r];
            }
            continue;
        }
#pragma unroll
        for (int step = 0; step < 2; ++step) {  // partner group: lane ^ 16, then lane ^ 32
            auto other = [&](float x) { return step == 0 ? lane_xor16(x) : lane_xor32(x); };
            const float mo = other(m[r]), lo = other(l[r]);
            float4 ao[DV];
#pragma unroll
            for (int u = 0; u < DV; ++u) {
                ao[u].x = other(acc[r][u].x);
                ao[u].y = other(acc[r][u].y);
                ao[u].z = other(acc[r][u].z);
                ao[u].w = other(acc[r][u].w);
            }
            fold_state<DV>(m[r], l[r], acc[r], mo, lo, ao);
        }
        if (grp == 0) {
#pragma unroll
            for (int u = 0; u < DV; ++u) wacc[wave][r][li + 16 * u] = acc[r][u];
            if (li == 0) {
                wml[wave][r][0] = m[r];
                wml[wave][r][1] = l[r];
            }
        }
    }
    __syncthreads();
    const uint64_t row_stride = kDecodePartStride + 4 * D4;
    float* part = g.ws + ((b * g.kv_heads + kvh) * P + p) * R * row_stride;
    if constexpr (NS == 16) {
        // the 16 states' weights exp(m_s - max) of each row, once: row r's
        // states sit in the 16-lane row r of waves 0 .. R / 4 (DPP rows)
        __shared__ float coef[RT][16];
        __shared__ float rml[RT][2];
        if (static_cast<uint32_t>(wave) * kWave < R * 16) {  // wave-uniform
            const uint32_t r = tid / 16, st = tid % 16;
            const float ms = r < R ? wml[st][r][0] : -INFINITY;
            const float mm = row_max(ms);
            const float cw = ms == -INFINITY ? 0.f : expf(ms - mm);
            const float ll = row_sum((r < R ? wml[st][r][1] : 0.f) * cw);
            if (r < R) {
                coef[r][st] = cw;
                if (st == 0) {
                    rml[r][0] = mm;
                    rml[r][1] = ll;
                }
            }
        }
        __syncthreads();
        for (uint32_t i = tid; i < R * D4; i += 256) {
            const uint32_t r = i / D4, c = i % D4;
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int w = 0; w < NS; ++w) a = f4_fma(coef[r][w], wacc[w][r][c], a);
            reinterpret_cast<float4*>(part + r * row_stride + kDecodePartStride)[c] = a;
            if (c == 0) {
                part[r * row_stride] = rml[r][0];
                part[r * row_stride + 1] = rml[r][1];
            }
        }
        return;
    }
    for (uint32_t i = tid; i < R * D4; i += 256) {
        const uint32_t r = i / D4, c = i % D4;
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < NS; ++w) mm = fmaxf(mm, wml[w][r][0]);
        float ll = 0.f;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        if (mm != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NS; ++w) {
                const float mw = wml[w][r][0];
                const float cw = mw == -INFINITY ? 0.f : expf(mw - mm);
                ll = fmaf(wml[w][r][1], cw, ll);
                a = f4_fma(cw, wacc[w][r][c], a);
            }
        }
        reinterpret_cast<float4*>(part + r * row_stride + kDecodePartStride)[c] = a;
        if (c == 0) {
            part[r * row_stride] = mm;
            part[r * row_stride + 1] = ll;
        }
    }
}

// Merges the P partials of one query row of a KV head: grid (kv_heads * R,
// batch), R = group * seq rows per KV head. Threads own float4 output slots,
// T = 256 / (head_dim / 4) threads per slot, each over every T-th partial;
// all of a thread's partial rows are loaded before the weights exp(m_p -
// max) / sum are worked out (one wave, from the (m, l) of every partial), so
// both wait on one memory round trip. The T sums of a slot are added in LDS
// in thread order.
constexpr int kMergeMaxParts = 64;

// The leading (preloaded) arguments locate the partials: the workspace,
// P partials per row, head_dim, R = group * seq rows per KV head, and the
// KV heads; the loads go out while the argument block is fetched.
// KP > 0: partials per thread, at least ceil(P / T); KP == 0: up to
// kMergeMaxParts / 4 per thread.
template <int KP>
__global__ __launch_bounds__(256) void attn_decode_merge(const float* ws, uint32_t P, uint32_t head_dim, uint32_t R,
                                                         uint32_t kv_heads, Geo g) {
    __shared__ float coef[kMergeMaxParts];
    __shared__ float4 red[256];
    const uint32_t D4 = head_dim / 4;
    const uint32_t kvh = blockIdx.x / R, r = blockIdx.x % R;
    const uint64_t b = blockIdx.y;
    const int tid = threadIdx.x, lane = tid % kWave;
    const uint64_t row_stride = kDecodePartStride + 4 * D4;
    const float* base = ws + (b * kv_heads + kvh) * P * R * row_stride;
    const uint32_t T = 256 / D4;  // threads per slot: 4 .. 16
    const uint32_t c = tid % D4, q = tid / D4;  // q >= T (head_dim 192): idle
    const bool mine = q < T;
    // (m, l) of partial `lane` (lanes past P re-read the last one), loaded
    // first: wave 0's weights below wait on these loads alone, while the
    // partial rows are still in flight
    const bool on = static_cast<uint32_t>(lane) < P;
    const float2 ml = *reinterpret_cast<const float2*>(
        base + static_cast<uint64_t>(min(static_cast<uint32_t>(lane), P - 1) * R + r) * row_stride);
    __builtin_amdgcn_sched_barrier(0);  // kept ahead of the row loads
    constexpr int kPer = KP > 0 ? KP : kMergeMaxParts / 4;
    float4 v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        if constexpr (KP > 0) {
            // unconditional (partials past P re-read the last one and are
            // skipped below), so no load waits at a branch's join
            const uint32_t pp = min(q + u * T, P - 1);
            v[u] = reinterpret_cast<const float4*>(base + (pp * R + r) * row_stride + kDecodePartStride)[c];
        } else {
            const uint32_t pp = q + u * T;
            v[u] = mine && pp < P
                       ? reinterpret_cast<const float4*>(base + (pp * R + r) * row_stride + kDecodePartStride)[c]
                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    if (tid < kWave) {
        const float mp = on ? ml.x : -INFINITY;
        const float lp = on ? ml.y : 0.f;
        const float mx = wave_max(mp);
        const float e = mp == -INFINITY ? 0.f : expf(mp - mx);
        const float total = wave_sum(lp * e);
        if (on) coef[lane] = e / total;
    }
    // the rest of the arguments (the outputs), in one batch of loads
    prefetch_kernarg<arg_bytes<const float*, uint32_t, uint32_t, uint32_t, uint32_t, Geo>()>();
    __syncthreads();
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const uint32_t pp = q + u * T;
        if (mine && pp < P) a = f4_fma(coef[pp], v[u], a);
    }
    red[tid] = a;
    __syncthreads();
    if (q != 0) return;
    for (uint32_t o = 1; o < T; ++o) {
        const float4 x = red[tid + o * D4];
        a.x += x.x;
        a.y += x.y;
        a.z += x.z;
        a.w += x.w;
    }
    const uint32_t S = g.seq, gi = r / S, t = r % S;
    const uint64_t h = kvh * g.group + gi;
    if (g.out != nullptr) reinterpret_cast<float4*>(g.out + ((b * g.heads + h) * S + t) * (4 * D4))[c] = a;
    // MergeHeads layout [B, S, H * D] (reference/layout.rs merge_heads)
    const uint64_t mrow = (b * S + t) * g.heads + h;
    if (g.merged != nullptr) reinterpret_cast<float4*>(g.merged + mrow * (4 * D4))[c] = a;
    if (g.mirror != nullptr) reinterpret_cast<float4*>(g.mirror + mrow * (4 * D4))[c] = a;
}

// ---- prefill: the f32 matrix cores ----
//
// A block owns 64 queries of one head (query wave w: queries 16 w .. 16 w +
// 15 of the block's range) and streams the keys 32 at a time; with KH = 2
// two waves serve each query wave, one per 16-key half of every tile, and
// their softmax states are combined through LDS at the end. Each
// tile of K and V rows goes to LDS (row stride D + 4 floats, so a wave's
// 16-byte K reads and 4-byte V reads hit 64 distinct banks) while the next
// tile's rows wait in registers. Per tile a wave forms S^T = K Q^T (keys x
// its 16 queries) and O^T += V^T P^T (dims x queries) with
// v_mfma_f32_16x16x4_f32: f32 products and f32 sums, like the VALU form.
// The accumulator layout puts rows 4 (l / 16) + i, column l % 16 in lane l,
// so every value a lane holds of S^T and O^T belongs to query l % 16: the
// online-softmax state (m, l) is per lane, a query's reductions span lanes
// l % 16 + 16 r (two lane swaps), and P^T is S^T's registers used as the B
// operand of the second product (the keys of its step i are 4 (l / 16) + i).
// The reduction over d is taken in a permuted order, the same for both
// operands: of each 16 dims, step s takes d = 4 (l / 16) + s, so a lane's
// operands of four steps are one float4 of K in LDS and of Q in registers.
// A block runs two query tiles one after the other, the last and the first,
// the second-to-last and the second, ..., so every block's causal key ranges
// add up to about the same work.
typedef float v4f_t __attribute__((ext_vector_type(4)));
constexpr int kPfQ = 64;  // queries per block
constexpr int kPfK = 32;  // keys per tile

// The next tile's K/V rows wait in registers while a tile is computed; they
// travel by value (PfRows). Filled through references into arrays, they were
// kept in scratch memory (at 128 registers per lane) or in LDS slots (at
// more), stored as soon as each load returned, so the loads never
// overlapped a tile's products. 8B layer at 1024 tokens, attn_prefill<128,
// 2>: 154.3 us in scratch, 129.1 in LDS slots, 106.0 in registers at two
// waves per SIMD (144 registers, one block per CU), 108.9 at four (128
// registers, two blocks per CU).
template <int N>
struct PfRows {
    float4 k[N], v[N];
};

template <int D, int KH>
__global__ __launch_bounds__(256 * KH) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_prefill(Geo g,
                                                                                                  uint32_t qtiles) {
    prefetch_kernarg<arg_bytes<Geo, uint32_t>()>();
    constexpr int NT = 256 * KH;             // threads
    constexpr int LS = D + 4;                // LDS row stride (floats)
    constexpr int D16 = D / 16;              // float4 of Q per lane, and 16-dim output tiles
    constexpr int F4 = kPfK * D / 4 / NT;    // float4 of K (and of V) per thread per tile
    constexpr int NS = 2 / KH;               // 16-key halves of a tile per wave
    static_assert(F4 >= 1 && KH >= 1 && KH <= 2, "tile split");
    __shared__ __align__(16) float ks[kPfK * LS];
    __shared__ __align__(16) float vs[kPfK * LS];
    // KH == 2: the second key half's softmax state (m, l, o) per lane of
    // each query wave, field-major
    constexpr int XF = 2 + D / 4;
    __shared__ float xs[KH == 2 ? XF * 256 : 1];
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const int qw = wave % 4;                 // query wave: queries 16 qw .. of the tile
    const int half = KH == 2 ? wave / 4 : 0; // KH == 2: keys 16 half .. 16 half + 15 of each tile
    const int c = lane % 16, kk = lane / 16;
    const uint32_t h = blockIdx.y;
    const uint64_t b = blockIdx.z;
    const uint32_t kvh = h / g.group;
    const uint32_t past = past_of(g);
    // query tiles qtiles - 1 - x, then x (the causal key ranges of the two
    // add up to about the same for every block)
    for (uint32_t pass = 0; pass < 2; ++pass) {
    const uint32_t qt = pass == 0 ? qtiles - 1 - blockIdx.x : blockIdx.x;
    if (pass == 1 && qt >= qtiles - 1 - blockIdx.x) break;  // block-uniform
    const uint32_t q0 = qt * kPfQ + qw * 16;    // the wave's first query
    const uint32_t t = q0 + c;                  // this lane's query
    const uint32_t tq = min(t, g.seq - 1);      // lanes past the end compute on the last query, unstored
    const uint32_t block_keys = past + min(g.seq, (qt + 1) * kPfQ);
    const uint32_t wave_keys = q0 < g.seq ? past + min(g.seq - 1, q0 + 15) + 1 : 0;
    const uint32_t my_keys = past + t + 1;

    float4 qv[D16];
    const float4* qrow = reinterpret_cast<const float4*>(g.q + ((b * g.heads + h) * g.seq + tq) * D);
#pragma unroll
    for (int j = 0; j < D16; ++j) qv[j] = qrow[4 * j + kk];
    v4f_t o[D16];
#pragma unroll
    for (int j = 0; j < D16; ++j) o[j] = v4f_t{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, lsum = 0.f;

    const uint64_t time_stride = static_cast<uint64_t>(g.kv_heads) * D;
    const float* kbase = g.cache + b * g.batch_stride + g.layer_offset + kvh * D;
    const float* vbase = kbase + g.parity_stride;
    // rows past the block's keys re-read its last key (their scores are
    // masked); the rows travel by value (an array the lambda filled through a
    // reference would be kept in memory, stored as soon as it arrived)
    auto load = [&](uint32_t kt) -> PfRows<F4> {
        PfRows<F4> n;
#pragma unroll
        for (int u = 0; u < F4; ++u) {
            const uint32_t e = tid + NT * u, row = e / (D / 4), col = e % (D / 4);
            const uint64_t j = min(kt + row, block_keys - 1);
            n.k[u] = reinterpret_cast<const float4*>(kbase + j * time_stride)[col];
            n.v[u] = reinterpret_cast<const float4*>(vbase + j * time_stride)[col];
        }
        return n;
    };
    PfRows<F4> nx = load(0);
    for (uint32_t kt = 0; kt < block_keys; kt += kPfK) {
        __syncthreads();  // every wave is done reading the previous tile
#pragma unroll
        for (int u = 0; u < F4; ++u) {
            const uint32_t e = tid + NT * u, row = e / (D / 4), col = e % (D / 4);
            *reinterpret_cast<float4*>(ks + row * LS + 4 * col) = nx.k[u];
            *reinterpret_cast<float4*>(vs + row * LS + 4 * col) = nx.v[u];
        }
        __syncthreads();
        // the next tile's rows, waiting in registers while this tile is computed
        nx = load(kt + kPfK);
        // wave-uniform: no key of the wave's part of the tile is visible to it
        if (kt + 16 * half >= wave_keys) continue;
        // S^T: keys 16 sub + 4 kk + i of the tile, query c
        v4f_t st[NS];
#pragma unroll
        for (int si = 0; si < NS; ++si) {
            const int sub = KH == 2 ? half : si;
            st[si] = v4f_t{0.f, 0.f, 0.f, 0.f};
            const float* krow = ks + (sub * 16 + c) * LS + 4 * kk;
#pragma unroll
            for (int j = 0; j < D16; ++j) {
                const float4 k4 = *reinterpret_cast<const float4*>(krow + 16 * j);
                st[si] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.x, qv[j].x, st[si], 0, 0, 0);
                st[si] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.y, qv[j].y, st[si], 0, 0, 0);
                st[si] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.z, qv[j].z, st[si], 0, 0, 0);
                st[si] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.w, qv[j].w, st[si], 0, 0, 0);
            }
        }
        float p[NS][4];
        float tmax = -INFINITY;
#pragma unroll
        for (int si = 0; si < NS; ++si)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int sub = KH == 2 ? half : si;
                const uint32_t key = kt + 16 * sub + 4 * kk + i;
                p[si][i] = key < my_keys ? st[si][i] * g.scale : -INFINITY;
                tmax = fmaxf(tmax, p[si][i]);
            }
        tmax = fmaxf(tmax, lane_xor16(tmax));
        tmax = fmaxf(tmax, lane_xor32(tmax));
        // With one key half per wave a query can see none of a tile's keys
        // (m_new == -inf): the guards keep corr and every weight 0, not NaN.
        // (With both halves key 0 is visible to every query, so m is finite
        // from the first tile on.)
        const float m_new = fmaxf(m, tmax);
        const float corr = m == -INFINITY ? 0.f : expf(m - m_new);
        float psum = 0.f;
#pragma unroll
        for (int si = 0; si < NS; ++si)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[si][i] = p[si][i] == -INFINITY ? 0.f : expf(p[si][i] - m_new);
                psum += p[si][i];
            }
        psum += lane_xor16(psum);
        psum += lane_xor32(psum);
        lsum = lsum * corr + psum;
        m = m_new;
        // O^T += V^T P^T: dims 16 j + c (A), keys 16 sub + 4 kk + i (k), query c (B)
#pragma unroll
        for (int j = 0; j < D16; ++j) {
            o[j] *= corr;
#pragma unroll
            for (int si = 0; si < NS; ++si)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int sub = KH == 2 ? half : si;
                    o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vs[(16 * sub + 4 * kk + i) * LS + 16 * j + c],
                                                                 p[si][i], o[j], 0, 0, 0);
                }
        }
    }
    if constexpr (KH == 2) {
        // the second half's state through LDS; the first half's waves merge
        const int x = qw * kWave + lane;
        if (half == 1) {
            xs[x] = m;
            xs[256 + x] = lsum;
#pragma unroll
            for (int j = 0; j < D16; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) xs[(2 + 4 * j + e) * 256 + x] = o[j][e];
        }
        __syncthreads();
        if (half == 1) continue;
        const float m1 = xs[x], l1 = xs[256 + x];
        const float mm = fmaxf(m, m1);
        const float c0 = m == -INFINITY ? 0.f : expf(m - mm), c1 = m1 == -INFINITY ? 0.f : expf(m1 - mm);
        lsum = lsum * c0 + l1 * c1;
#pragma unroll
        for (int j = 0; j < D16; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[j][e] = o[j][e] * c0 + xs[(2 + 4 * j + e) * 256 + x] * c1;
    }
    if (t < g.seq) {
        const float inv = 1.0f / lsum;
        // [B, H, S, D], and MergeHeads' [B, S, H * D] (fused form)
        float* orow = g.out != nullptr ? g.out + ((b * g.heads + h) * g.seq + t) * D + 4 * kk : nullptr;
        float* mrow = g.merged != nullptr ? g.merged + ((b * g.seq + t) * g.heads + h) * D + 4 * kk : nullptr;
#pragma unroll
        for (int j = 0; j < D16; ++j) {
            const float4 v = make_float4(o[j][0] * inv, o[j][1] * inv, o[j][2] * inv, o[j][3] * inv);
            if (orow != nullptr) *reinterpret_cast<float4*>(orow + 16 * j) = v;
            if (mrow != nullptr) *reinterpret_cast<float4*>(mrow + 16 * j) = v;
        }
    }
    }
}

// ---- prefill, fused form: SplitHeads, Rope and KvAppend in one pass ----
//
// One block per token (b, t) of the chunk: the pair angles' sine and cosine
// for its position (f64, as rope_vec4 and reference/rope.rs compute them,
// once per token), then q [b, t, H * D] rotated into qr [b, h, t, D] (the
// attention's input), k [b, t, Hkv * D] rotated into the cache's K row of
// slot past + t, and v copied into its V row (reference/attention.rs:33-83).
// Rotation x c - y s, x s + y c in f32, the expressions of rope_vec4: the
// results equal the unfused ops' bit for bit.
template <int D>
__global__ __launch_bounds__(256) void prefill_prep(Geo g, float* __restrict__ qr) {
    prefetch_kernarg<arg_bytes<Geo, float*>()>();
    __shared__ float sc[D];  // [D / 2] sine, [D / 2] cosine
    constexpr uint32_t D4 = D / 4;
    const uint32_t S = g.seq, H = g.heads, Hkv = g.kv_heads;
    const uint64_t bt = blockIdx.x, b = bt / S, t = bt % S;
    const uint32_t past = past_of(g);
    const double position = static_cast<double>(g.pos[bt]);
    for (uint32_t pair = threadIdx.x; pair < D / 2; pair += blockDim.x) {
        const double exponent = 2.0 * static_cast<double>(pair) / static_cast<double>(D);
        const double angle = position / pow(g.theta, exponent);
        sc[pair] = static_cast<float>(sin(angle));
        sc[D / 2 + pair] = static_cast<float>(cos(angle));
    }
    __syncthreads();
    const bool neox = g.rope_variant == SL_ROPE_NEOX;
    // items per head: NeoX the float4 c < D / 8 with its partner c + D / 8
    // (pairs d, d + D / 2), GPT-J every float4 (pairs 2i, 2i + 1)
    const uint32_t per_head = neox ? D / 8 : D4;
    // rotates item c of the head row src into dst (float4 indices)
    auto rotate_item = [&](const float4* src, float4* dst, uint32_t c) {
        if (neox) {
            const float4 x = src[c], y = src[c + D / 8];
            const uint32_t p0 = 4 * c;
            const float s0 = sc[p0], s1 = sc[p0 + 1], s2 = sc[p0 + 2], s3 = sc[p0 + 3];
            const float c0 = sc[D / 2 + p0], c1 = sc[D / 2 + p0 + 1], c2 = sc[D / 2 + p0 + 2], c3 = sc[D / 2 + p0 + 3];
            dst[c] = make_float4(x.x * c0 - y.x * s0, x.y * c1 - y.y * s1, x.z * c2 - y.z * s2, x.w * c3 - y.w * s3);
            dst[c + D / 8] = make_float4(x.x * s0 + y.x * c0, x.y * s1 + y.y * c1, x.z * s2 + y.z * c2,
                                         x.w * s3 + y.w * c3);
        } else {
            const float4 a = src[c];
            const float s0 = sc[2 * c], c0 = sc[D / 2 + 2 * c], s1 = sc[2 * c + 1], c1 = sc[D / 2 + 2 * c + 1];
            dst[c] = make_float4(a.x * c0 - a.y * s0, a.x * s0 + a.y * c0, a.z * c1 - a.w * s1, a.z * s1 + a.w * c1);
        }
    };
    const float4* qrow = reinterpret_cast<const float4*>(g.q + bt * H * D);
    for (uint32_t i = threadIdx.x; i < H * per_head; i += blockDim.x) {
        const uint32_t h = i / per_head, c = i % per_head;
        rotate_item(qrow + h * D4, reinterpret_cast<float4*>(qr + ((b * H + h) * S + t) * D), c);
    }
    float* krow = g.wcache + b * g.batch_stride + g.layer_offset + static_cast<uint64_t>(past + t) * Hkv * D;
    const float4* ksrc = reinterpret_cast<const float4*>(g.k_new + bt * Hkv * D);
    for (uint32_t i = threadIdx.x; i < Hkv * per_head; i += blockDim.x) {
        const uint32_t h = i / per_head, c = i % per_head;
        rotate_item(ksrc + h * D4, reinterpret_cast<float4*>(krow + h * D), c);
    }
    const float4* vsrc = reinterpret_cast<const float4*>(g.v_new + bt * Hkv * D);
    float4* vrow = reinterpret_cast<float4*>(krow + g.parity_stride);
    for (uint32_t i = threadIdx.x; i < Hkv * D4; i += blockDim.x) vrow[i] = vsrc[i];
}

}  // namespace

namespace {

Geo make_geo(const AttentionArgs& a, const Workspace& ws) {
    Geo g{};
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
    g.dyn = a.dyn;
    g.pos = a.positions;
    g.theta = static_cast<double>(a.theta);
    g.rope_variant = a.rope_variant;
    g.merged = a.merged;
    g.mirror = a.mirror;
    g.q_split = a.q_split;
    g.k_split = a.k_split;
    g.v_split = a.v_split;
    g.q_rot = a.q_rot;
    g.k_rot = a.k_rot;
    g.rope_tab = a.rope_table;
    if (a.block_table != nullptr) {  // paged cache: a pool of pages, rows at their own lengths
        const uint64_t row = a.kv_heads * a.head_dim;
        g.parity_stride = static_cast<uint64_t>(a.page_size) * row;
        g.page_stride = 2 * g.parity_stride;
        g.layer_offset = a.layer * a.num_pages * g.page_stride;
        g.batch_stride = 0;
        g.block_table = a.block_table;
        g.seq_past = a.seq_lens;
        g.page_size = a.page_size;
        g.pages_per_seq = a.pages_per_seq;
    }
    return g;
}

// Partials per (row, KV head): one per 128 positions of max_seq (64 for
// head_dim 64, whose waves then take 8-key tiles), at most kMergeMaxParts,
// and no more than keep the grid near kDecodeGridBlocks blocks. Each
// block's share is latency-bound (one or two tiles per wave), so a batch of
// many sequences is better served by fewer, longer partials than by rounds
// of short blocks (8B, batch 8: 2,022 tok/s at 512 blocks, 2,006 at 1024,
// 1,946 with 32 partials as at batch 1). Half the positions per partial and
// 8-key tiles at head_dim 64: 1B decode 1,860-1,881 -> 1,884-1,897 tok/s;
// the same at head_dim 128: 8B 670-674 -> 665-668. Shapes only: the grid
// never depends on past_len.
constexpr uint64_t kDecodeGridBlocks = 512;
uint64_t decode_part_span(const AttentionArgs& a) { return a.head_dim == 64 ? 64 : 128; }
uint64_t decode_parts(const AttentionArgs& a) {
    uint64_t parts = (a.max_seq + decode_part_span(a) - 1) / decode_part_span(a);
    const uint64_t rows = a.batch * a.kv_heads;
    const uint64_t by_grid = rows ? (kDecodeGridBlocks + rows - 1) / rows : 1;
    if (parts > by_grid) parts = by_grid;
    if (parts < 1) parts = 1;
    return parts > kMergeMaxParts ? kMergeMaxParts : parts;
}

// The decode kernels (tile + merge); hipErrorNotSupported for shapes they
// do not take (nothing launched).
hipError_t launch_decode(const AttentionArgs& a, Geo g, const Workspace& ws, hipStream_t s, bool fused,
                         bool paged = false) {
    const uint64_t rows = static_cast<uint64_t>(g.group) * a.seq;
    const uint64_t dv = a.head_dim / 64;
    const uint64_t rt = rows <= 4 ? 4 : rows <= 8 ? 8 : 16;
    const uint64_t parts = decode_parts(a);
    const bool aligned = aligned16(a.q) && aligned16(a.k_new) && aligned16(a.v_new) && aligned16(a.cache) &&
                         (a.out == nullptr || aligned16(a.out)) && (a.merged == nullptr || aligned16(a.merged)) &&
                         (a.mirror == nullptr || aligned16(a.mirror));
    if (!(rows <= kDecodeMaxRows && a.head_dim % 64 == 0 && dv >= 1 && dv <= 4 && rt * dv <= 32 && aligned &&
          a.batch * a.kv_heads * parts * rows * (kDecodePartStride + a.head_dim) <= ws.floats))
        return hipErrorNotSupported;
    if (fused && (a.positions == nullptr || (a.rope_variant == SL_ROPE_NEOX && dv % 2 != 0 && dv != 1) ||
                  a.rope_variant > SL_ROPE_GPTJ))
        return hipErrorNotSupported;
    g.chunks = static_cast<uint32_t>(parts);
    g.chunk = kDecodeTile;
    const dim3 grid(static_cast<unsigned>(parts), g.kv_heads, static_cast<unsigned>(a.batch));
    const size_t lds = fused ? a.seq * a.head_dim * sizeof(float) : 0;
    const uint32_t* past_src = paged ? g.seq_past : g.dyn;
#define SL_DECODE_ARGS past_src, g.past_len, g.q, g.seq, g.group, g.heads, g
#define SL_DECODE_K(DVv, RTv, K)                                                                      \
    (fused ? (paged ? attn_decode<DVv, RTv, true, true, K><<<grid, 256, lds, s>>>(SL_DECODE_ARGS)     \
                    : attn_decode<DVv, RTv, true, false, K><<<grid, 256, lds, s>>>(SL_DECODE_ARGS))   \
     : paged ? attn_decode<DVv, RTv, false, true, K><<<grid, 256, lds, s>>>(SL_DECODE_ARGS)           \
             : attn_decode<DVv, RTv, false, false, K><<<grid, 256, lds, s>>>(SL_DECODE_ARGS))
    // 8-key tiles at head_dim 64, and at 128 where the partials were capped
    // by the grid size (batch 8, 8B: 2,617-2,624 -> 2,689-2,690 tok/s; at
    // batch 1, with the partials unchanged, they cost 642-644 -> 629-634)
    const bool short_tiles =
        dv == 1 || (dv == 2 && parts < (a.max_seq + decode_part_span(a) - 1) / decode_part_span(a));
#define SL_DECODE(DVv, RTv) (short_tiles ? SL_DECODE_K(DVv, RTv, 2) : SL_DECODE_K(DVv, RTv, 4))
#define SL_DECODE_LONG(DVv, RTv) SL_DECODE_K(DVv, RTv, 4)
    switch (dv * 100 + rt) {
        case 104: SL_DECODE(1, 4); break;
        case 108: SL_DECODE(1, 8); break;
        case 116: SL_DECODE(1, 16); break;
        case 204: SL_DECODE(2, 4); break;
        case 208: SL_DECODE(2, 8); break;
        case 216: SL_DECODE(2, 16); break;
        case 304: SL_DECODE_LONG(3, 4); break;
        case 308: SL_DECODE_LONG(3, 8); break;
        case 404: SL_DECODE_LONG(4, 4); break;
        default: SL_DECODE_LONG(4, 8); break;
    }
#undef SL_DECODE
#undef SL_DECODE_LONG
#undef SL_DECODE_K
#undef SL_DECODE_ARGS
    // partials per merge thread (T = 256 / (head_dim / 4) threads per float4
    // slot, each over every T-th partial): up to four, the unconditional
    // form with exactly that many loads; more, the guarded form
    const uint64_t T = 256 / (a.head_dim / 4), per = (parts + T - 1) / T;
    const dim3 mgrid(g.kv_heads * static_cast<unsigned>(rows), static_cast<unsigned>(a.batch));
#define SL_MERGE(KP) \
    attn_decode_merge<KP><<<mgrid, 256, 0, s>>>(g.ws, static_cast<uint32_t>(parts), g.head_dim, static_cast<uint32_t>(rows), g.kv_heads, g)
    if (per <= 1) SL_MERGE(1);
    else if (per <= 2) SL_MERGE(2);
    else if (per <= 4) SL_MERGE(4);
    else SL_MERGE(0);
#undef SL_MERGE
    return hipGetLastError();
}

}  // namespace

hipError_t launch_rope_sincos(const uint32_t* positions, uint64_t tokens, uint64_t head_dim, float theta,
                              float* table, hipStream_t s) {
    if (tokens == 0) return hipSuccess;
    if (head_dim % 2 != 0 || tokens * head_dim > 0xffffffffull) return hipErrorInvalidValue;
    const uint64_t n = tokens * (head_dim / 2);
    rope_sincos<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(
        positions, static_cast<uint32_t>(tokens), static_cast<uint32_t>(head_dim), static_cast<double>(theta), table);
    return hipGetLastError();
}

uint64_t attention_workspace_floats(const AttentionArgs& a) {
    const uint64_t rows = a.heads / (a.kv_heads ? a.kv_heads : 1) * a.seq;
    return a.batch * a.kv_heads * decode_parts(a) * rows * (kDecodePartStride + a.head_dim);
}

bool attention_fused_prefill(const AttentionArgs& a) {
    const uint64_t rows = a.heads / (a.kv_heads ? a.kv_heads : 1) * a.seq;
    const uint64_t dv = a.head_dim / 64;
    const uint64_t rt = rows <= 4 ? 4 : rows <= 8 ? 8 : 16;
    return !(rows <= kDecodeMaxRows && a.head_dim % 64 == 0 && dv >= 1 && dv <= 4 && rt * dv <= 32);
}

uint64_t attention_fused_workspace_floats(const AttentionArgs& a) {
    return attention_fused_prefill(a) ? a.batch * a.seq * a.heads * a.head_dim : attention_workspace_floats(a);
}

hipError_t launch_paged_attention(const PagedAttentionArgs& p, const Workspace& ws, hipStream_t s) {
    AttentionArgs a{p.q, p.k_new, p.v_new, p.pool, p.out, p.batch, p.layers, p.layer, p.heads, p.kv_heads, 1,
                    0, p.head_dim, static_cast<uint64_t>(p.pages_per_seq) * p.page_size, p.scale, nullptr};
    if (a.batch * a.heads == 0 || a.head_dim == 0 || a.kv_heads == 0 || p.page_size % kDecodeTile != 0)
        return hipErrorNotSupported;
    a.block_table = p.block_table;
    a.seq_lens = p.seq_lens;
    a.num_pages = p.num_pages;
    a.page_size = p.page_size;
    a.pages_per_seq = p.pages_per_seq;
    return launch_decode(a, make_geo(a, ws), ws, s, false, true);
}

uint64_t paged_attention_workspace_floats(const PagedAttentionArgs& p) {
    AttentionArgs a{};
    a.batch = p.batch;
    a.heads = p.heads;
    a.kv_heads = p.kv_heads;
    a.seq = 1;
    a.head_dim = p.head_dim;
    a.max_seq = static_cast<uint64_t>(p.pages_per_seq) * p.page_size;
    return attention_workspace_floats(a);
}

hipError_t launch_attention_fused(const AttentionArgs& a, const Workspace& ws, hipStream_t s) {
    if (a.batch * a.heads * a.seq == 0 || a.head_dim == 0 || a.kv_heads == 0) return hipErrorNotSupported;
    const bool paged = a.block_table != nullptr;
    if (paged && (a.seq != 1 || a.page_size % kDecodeTile != 0)) return hipErrorNotSupported;
    const hipError_t d = launch_decode(a, make_geo(a, ws), ws, s, true, paged);
    if (d != hipErrorNotSupported || paged) return d;
    // Prefill: prefill_prep (SplitHeads, Rope, KvAppend), then attn_prefill
    // writing the attention output and / or MergeHeads' layout. The rotated q
    // goes to q_rot when set (the caller's staging area, which nothing the
    // kernels read or write overlaps), else to the workspace; the unit's
    // other intermediates must be dead (no staging) and the output
    // projection not chained.
    const uint64_t qr_floats = a.batch * a.seq * a.heads * a.head_dim;
    const bool aligned = aligned16(a.q) && aligned16(a.k_new) && aligned16(a.v_new) && aligned16(a.cache) &&
                         (a.out == nullptr || aligned16(a.out)) && (a.merged == nullptr || aligned16(a.merged)) &&
                         (a.q_rot == nullptr || aligned16(a.q_rot));
    if (a.seq < 16 || !(a.head_dim == 64 || a.head_dim == 128) || !aligned || a.positions == nullptr ||
        a.rope_variant > SL_ROPE_GPTJ || a.mirror != nullptr || a.q_split != nullptr || a.k_split != nullptr ||
        a.v_split != nullptr || a.k_rot != nullptr || (a.out == nullptr && a.merged == nullptr) ||
        (a.q_rot == nullptr && qr_floats > ws.floats) || a.batch * a.seq > 0x7fffffffull)
        return hipErrorNotSupported;
    float* qr = a.q_rot != nullptr ? a.q_rot : ws.data;
    Geo g = make_geo(a, ws);
    const unsigned tokens = static_cast<unsigned>(a.batch * a.seq);
    if (a.head_dim == 64) prefill_prep<64><<<tokens, 256, 0, s>>>(g, qr);
    else prefill_prep<128><<<tokens, 256, 0, s>>>(g, qr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    g.q = qr;
    const uint32_t qtiles = static_cast<uint32_t>((a.seq + kPfQ - 1) / kPfQ);
    const dim3 grid((qtiles + 1) / 2, g.heads, static_cast<unsigned>(a.batch));
    if (a.head_dim == 64) attn_prefill<64, 2><<<grid, 512, 0, s>>>(g, qtiles);
    else attn_prefill<128, 2><<<grid, 512, 0, s>>>(g, qtiles);
    return hipGetLastError();
}

hipError_t launch_attention(const AttentionArgs& a, const Workspace& ws, hipStream_t s) {
    const uint64_t queries = a.batch * a.heads * a.seq;
    if (queries == 0 || a.head_dim == 0) return hipSuccess;
    AttentionArgs plain = a;  // the unfused op writes only `out`
    plain.positions = nullptr;
    plain.merged = nullptr;
    plain.mirror = nullptr;
    Geo g = make_geo(plain, ws);

    // Decode path: kv_append fused into the tile kernel, then the merge.
    const hipError_t d = launch_decode(a, g, ws, s, false);
    if (d != hipErrorNotSupported) return d;

    hipError_t e = launch_kv_append(a.k_new, a.v_new, a.cache, a.batch, a.layers, a.layer, a.kv_heads, a.head_dim,
                                    a.max_seq, a.past_len, a.seq, a.dyn, s);
    if (e != hipSuccess) return e;
    const bool aligned = aligned16(a.q) && aligned16(a.cache) && aligned16(a.out);
    if (a.seq >= 16 && aligned && (a.head_dim == 64 || a.head_dim == 128)) {
        const uint32_t qtiles = static_cast<uint32_t>((a.seq + kPfQ - 1) / kPfQ);
        dim3 grid((qtiles + 1) / 2, g.heads, static_cast<unsigned>(a.batch));
        if (a.head_dim == 64) attn_prefill<64, 2><<<grid, 512, 0, s>>>(g, qtiles);
        else attn_prefill<128, 2><<<grid, 512, 0, s>>>(g, qtiles);
        return hipGetLastError();
    }
    if (a.head_dim > 256) return hipErrorInvalidValue;

    // Split the longest possible key range (max_seq, so the launch does not
    // depend on past_len) so that about 2048 waves run, each chunk holding
    // at least 64 keys, within the workspace; chunks past the current length
    // leave empty partials.
    const uint64_t max_keys = a.max_seq;
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

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_attention() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&attn_split<1>));
}

}  // namespace slhip
