// Group-quantized GEMV for decode (m <= 16 activation rows, m * k <= 16384)
// with the K reduction kept inside one workgroup, and the fusions a decoder
// layer wants around it.
//
// Arithmetic is the int8-limb MFMA scheme of qgemv_mfma.hip (exact integer
// products, one f32 combination per group; the weight tiles are the same
// QuantLayout::Mfma superblocks). What differs is the work split:
//  * a block of 8 waves owns one 16-row tile (or, for a gate/up pair, one
//    tile of each with 4 waves apiece) and the whole K range; its waves take
//    contiguous, group-aligned runs of superblocks and start their weight
//    loads (4 superblocks, rolling) before the activation prologue, then
//    add their partial sums in LDS in wave order. The group scales come
//    with each superblock's codes, or (long streams at m = 1) are loaded
//    into LDS for all the block's tiles at launch.
//    No split partials in HBM, no second launch, deterministic. Blocks stay
//    resident over several tiles (at most two per CU), so the prologue is
//    paid once per block, and the per-tile LDS sums are double-buffered;
//  * the activations are converted once per block from registers: every
//    thread holds its share of the m x k input as float4; the exponent of
//    each 256-element chunk comes from one wave's DPP max (no block-wide
//    pass), and only the RMSNorm sum of squares goes wave -> LDS -> row;
//  * up to three weights that read the same input run as one launch (q/k/v);
//  * prologue RMSNorm: x = (a * inv) * gamma with inv = 1/sqrt(ss/k + eps)
//    (reference/norm.rs:27-60), block 0 also writes x as the norm's output;
//  * epilogues: plain; residual (out2 = resid + out, reference/add.rs); pair
//    (h = silu(g) * u over a gate and an up tile, reference/swiglu.rs:40-84).
#include "common.h"
#include "kernels.h"
#include "starlight_hip.h"

#include <type_traits>

namespace slhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Calls f(std::integral_constant<int, I>) for I = 0 .. N-1, unrolled.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for_from(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for_from<I + 1, N>(f);
    }
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_from<0, N>(f);
}

// p, read into scalar registers: the value is wave-uniform by construction,
// and the compiler can no longer turn a per-lane choice among such values
// into a load from a per-lane address.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// p as a global-memory pointer: accesses through a pointer rebuilt from
// integers are otherwise flat, and a flat load makes the compiler wait for
// every outstanding load wherever it waits for this one.
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* global_ptr(T* p) {
    return (__attribute__((address_space(1))) T*)p;
}

// a0, a1 or a2 for si = 0, 1, 2 (si per lane), as two selects
template <typename T>
__device__ __forceinline__ T pick3(uint32_t si, T a0, T a1, T a2) {
    const T r = si >= 1 ? a1 : a0;
    return si >= 2 ? a2 : r;
}

// W waves per block (8 or 16); each thread holds at most kMaxF4 float4 of
// activations (F4: this launch's count), so a block holds max_elems(W).
// Bytes between consecutive rows of the limb matrices beyond k: the A
// operand of a 64-k step reads the same 16-byte columns of several rows,
// and rows a multiple of the bank width apart would all hit the same banks.
constexpr uint32_t kLimbPad = 64;
constexpr int kMaxF4 = 8;  // float4 of activations per thread, at most
constexpr int kWindow = 4;  // superblocks in flight per wave
constexpr int kSmStream = 0, kSmLds = 1, kSmOneRound = 2;  // stream modes (qgemv_fused's SM)
// activations a block holds: 16384 with 8 waves, 32768 with 16
constexpr uint32_t max_elems(int w) { return static_cast<uint32_t>(w) * kWave * 4 * kMaxF4; }
// float4 of scales each thread loads at launch: a block's tiles hold at
// most this many per thread (more spills registers: pair kernels hold one
// per group of a superblock, INT8 two, INT4 four at group 64). Every slot
// is loaded (unused ones re-read a used float4), and each wave64 load
// returns 1 KB to registers, so INT4 at one group per superblock keeps one
// slot: [14336 x 4096] 8.43-8.47 -> 8.31-8.37 us against four.
constexpr int qgemv_scale_slots(int nt, int gps, int bits) { return nt == 2 ? gps : bits == 4 ? (gps == 1 ? 1 : 4) : 2; }
// static LDS of the kernel with W waves: red, row_val, cfac, wres
constexpr size_t static_lds(int w) { return sizeof(float) * (kMaxF4 * w + 16 + max_elems(w) / 256 + 2 * w * 16 * 16); }

struct Seg {
    const uint8_t* tiles;
    const float* tscales;  // [tile][group][16]
    float* out;
    const float* resid;
    float* out2;
    uint32_t n, tile0;
};

struct Args {
    float* normed;
    float eps;
    Seg seg[kFusedMaxSegs];
    uint32_t nseg;
    uint32_t m, k, group, unit, sb_total, groups_total, sb_per_wave;
    uint32_t tiles_total;  // block tiles (pair mode: gate tiles)
    uint32_t epilogue;
    uint32_t tile_slots;   // tiles one block holds at most (LDS areas are sized for it)
    // Divisions by per-launch values, worked out by the launcher (a division
    // by a run-time value is about 15 instructions, and the prologue runs
    // at four waves per SIMD, so its instruction count is its length):
    // block b holds tiles_base + (b < tiles_rem) tiles; i / len = (i *
    // len_magic) >> 16 for i < 64; e / m = (e * m_magic) >> 16 for e < 4096;
    // f / run4 = mulhi(f, run4_magic) (run4 >= 8). Each exact over its range
    // (magic16(d) = ceil(2^16 / d), run4_magic = ceil(2^32 / run4)).
    uint32_t tiles_base, tiles_rem, len_magic, m_magic, run4_magic;
};

// ceil(2^16 / d): (n * magic16(d)) >> 16 == n / d for n < 2^16 / (d * ...)
// within the ranges the kernel uses (checked exhaustively: n < 64 for d <=
// 64, n < 128 for d <= 128, n < 4096 for d <= 16)
constexpr uint32_t magic16(uint32_t d) { return (65536u + d - 1) / d; }
// float4 of scales per tile and segment (sb_total superblocks, gps groups each)
constexpr uint32_t run4_of(uint32_t sb_total, uint32_t gps) { return sb_total * 16 * gps / 4; }


// One weight superblock of a wave's stream: its codes, 16 bytes per lane
// (INT8: two loads), and unless the scales of the block's tiles wait in LDS,
// the scales of its groups for the lane's row (s1: the second group of a
// superblock, group 64 only).
template <int BITS>
struct Item {
    uint4 c0, c1;
    float s0, s1;
};

// SPG: 64-k steps per group (1: group 64, 2: group 128, 0: a multiple of 256,
// counted at run time). LR (m <= 4): the three limbs of every activation row
// share one MFMA as its A rows 4 * m + limb, so a 64-k step is one LDS read
// and one MFMA; otherwise (m <= 16) each limb matrix is an MFMA of its own.
// SLICED: k is cut into gridDim.y slices of p.k columns; slice y = blockIdx.y
// reads columns [y p.k, (y + 1) p.k) of activation rows gridDim.y p.k / 4
// float4 apart, superblocks y p.sb_total .. of tiles holding gridDim.y
// p.sb_total, and writes its partial sums m n floats after slice y - 1's
// (the launcher adds the slices up). Every slice geometry follows from the
// grid, so the arguments are the same as for one slice.
// SM, how a wave streams its superblocks:
//  * kSmStream: each superblock's scales load with its codes, and the
//    window is refilled as it is consumed (past the stream's end with the
//    last superblock again, so that every wait stays one item deep);
//  * kSmLds: the scales of the block's tiles are loaded into LDS at launch
//    (one load per thread or a few, before the code window) instead of with
//    each superblock's codes; that pays where a wave streams more
//    superblocks than its window holds, and costs a dependent load before
//    the prologue's barrier where it does not;
//  * kSmOneRound: the whole stream fits the first window (no refills; those
//    would all re-read the last superblock, 1 KB of returns per wave each).
// The activations a, the RMSNorm weight gamma (null: no norm) and the
// m x k shape lead the arguments: the library is built to preload leading
// scalar arguments into scalar registers, so the activation loads go out
// at once, while the argument block is still being fetched. mk packs m
// (bits 0-4) and magic16(k / 256) (from bit 5), which finds a run's row.
template <int BITS, int NT, int SPG, bool LR, int F4, int W, bool SLICED, int SM>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(4))) void qgemv_fused(
    const float* __restrict__ a_in, const float* __restrict__ gamma, uint32_t mk, uint32_t k_in, Args p) {
    constexpr int kThreads = W * kWave, kWaves = W;
    static_assert(F4 <= kMaxF4, "activations per thread beyond the block's budget");
    constexpr int GPS = SPG == 1 ? 2 : 1;
    constexpr int PF = kWindow;
    constexpr bool LS = SM == kSmLds;
    constexpr int WPT = kWaves / NT;  // waves per tile
    constexpr uint32_t SB_BYTES = BITS == 4 ? 1024 : 2048;
    // [3][m][k + kLimbPad] limbs, tres [tile_slots][16][m] results, and
    // with LS tsc [tile_slots][NT][sb][16][gps] scales
    extern __shared__ __align__(16) int8_t limbs[];
    __shared__ float red[kMaxF4][kWaves];
    __shared__ float row_val[16];
    __shared__ float cfac[max_elems(W) / 256];  // per 256-element chunk: 2^(E-22)
    __shared__ float wres[2][kWaves][16][16];

    const int tid = threadIdx.x, lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform, kept in scalar registers
    const uint32_t M = mk & 31u, K = k_in, K4 = K / 4;
    const uint32_t ks = SLICED ? blockIdx.y : 0u;  // k slice
    const float* const a_slice = SLICED ? a_in + static_cast<uint64_t>(ks) * K : a_in;
    const uint32_t a_stride4 = SLICED ? gridDim.y * K4 : K4;
    const uint32_t RS = K + kLimbPad;  // limb row stride
    float* tres = reinterpret_cast<float*>(limbs + 3 * M * RS);
    float* tsc = tres + 16 * M * p.tile_slots;

    // ---- activations first, from the leading arguments alone (the
    // prologue waits for them only): element float4 f = tid + kThreads * u
    // of [m][k/4] ----
    const uint32_t total4 = M * K4;
    // k % 256 == 0 keeps a wave's 64 float4 inside one row: run (u, wave)
    // starts at float4 fb = wave * 64 + u * kThreads, row ru[u] = fb / k4
    // (both multiples of 64: (fb / 64) / (k / 256), fb / 64 < 128),
    // column cb[u] = fb % k4, all wave-uniform (a wave past the end takes
    // the last run), so no lane divides.
    uint32_t ru[F4], cb[F4];
#pragma unroll
    for (int u = 0; u < F4; ++u) {
        const uint32_t fb = min(static_cast<uint32_t>(wave * kWave + kThreads * u), total4 - kWave);
        ru[u] = __builtin_amdgcn_readfirstlane(((fb >> 6) * (mk >> 5)) >> 16);
        cb[u] = fb - ru[u] * K4;
    }
    float4 v[F4], gv[F4];
#pragma unroll
    for (int u = 0; u < F4; ++u) {
        if (kThreads * u < total4) {  // block-uniform: runs past the input load nothing
            const uint32_t c4 = cb[u] + lane;
            // rows of a k slice are a_stride4 float4 apart
            v[u] = reinterpret_cast<const float4*>(a_slice)[ru[u] * a_stride4 + c4];
            if (gamma != nullptr) gv[u] = reinterpret_cast<const float4*>(gamma)[c4];
        } else {
            v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    // the rest of the arguments, in one batch of loads (the activations are in flight)
    prefetch_kernarg<arg_bytes<const float*, const float*, uint32_t, uint32_t, Args>()>();
    const uint32_t sb_stride = SLICED ? gridDim.y * p.sb_total : p.sb_total;

    // ---- this wave's stream: for each block tile j (global tile
    // blockIdx.x + j * gridDim.x) the superblocks [sbA, sbA + len); every
    // wave has the same item count, so the per-tile barriers line up ----
    const int slot = wave / WPT, wi = wave % WPT;
    const uint32_t len = p.sb_per_wave;
    const uint32_t sbA = wi * len;
    // tiles blockIdx.x + j * gridDim.x: tiles_total / gridDim.x each, one
    // more for the first tiles_total % gridDim.x blocks
    const uint32_t my_tiles = p.tiles_base + (blockIdx.x < p.tiles_rem ? 1u : 0u);
    const uint32_t items = my_tiles * len;
    constexpr uint32_t gps = GPS;  // groups per superblock: 2 for group 64, else 1

    // Segment fields are read by constant index and chosen with selects: a
    // runtime index into the argument block (or a struct copy) would turn
    // every access into a dependent memory load.
    // First tiles of segments 1 and 2 (past the end when absent), as
    // scalars: a per-lane p.seg[si] would copy the argument block to scratch
    // memory to index it. The choices below are two selects each: written as
    // a nested conditional on a per-lane value, they compiled to branches.
    const uint32_t t1 = __builtin_amdgcn_readfirstlane(p.nseg > 1 ? p.seg[1].tile0 : 0xffffffffu);
    const uint32_t t2 = __builtin_amdgcn_readfirstlane(p.nseg > 2 ? p.seg[2].tile0 : 0xffffffffu);
    auto seg_of = [&](uint32_t t, uint32_t& tile) -> uint32_t {
        uint32_t si;
        if (NT == 1) {
            const bool g1 = t >= t1, g2 = t >= t2;
            si = (g1 ? 1u : 0u) + (g2 ? 1u : 0u);
            uint32_t off = g1 ? t1 : 0u;
            off = g2 ? t2 : off;
            tile = t - off;
        } else {
            si = static_cast<uint32_t>(slot);
            tile = t;
        }
        return si;
    };
    // The output-side fields are chosen per thread in the epilogue (and for
    // the residual prefetch); inside that divergent code a choice among
    // argument fields compiles to vector loads of the argument block, one
    // more memory round trip, so they are held in scalar registers here.
    float* s_out[kFusedMaxSegs];
    float* s_out2[kFusedMaxSegs];
    const float* s_res[kFusedMaxSegs];
    uint32_t s_n[kFusedMaxSegs];
#pragma unroll
    for (uint32_t i = 0; i < kFusedMaxSegs; ++i) {
        s_out[i] = uniform_ptr(SLICED ? p.seg[i].out + static_cast<uint64_t>(ks) * M * p.seg[i].n : p.seg[i].out);
        s_out2[i] = uniform_ptr(p.seg[i].out2);
        s_res[i] = uniform_ptr(p.seg[i].resid);
        s_n[i] = __builtin_amdgcn_readfirstlane(p.seg[i].n);
    }
#define SEG_PICK(a, si) pick3(si, a[0], a[1], a[2])
    // The stream as a table: lane l of the wave holds item l's weight and
    // scale addresses and its meta word (superblock along k, live flag,
    // last-of-tile flag), worked out once here in parallel; the loop then
    // reads item k's entries with v_readlane, keeping the shared scalar
    // unit's work per item small. A wave has at most 64 items (the launch
    // caps tiles per block to fit). Every item issues the same loads (the
    // dead superblocks of a trailing wave, and the window's fetches past the
    // stream's end, re-read a live one), so each wait is for one item only.
    const uint32_t nlive = sbA < p.sb_total ? min(len, p.sb_total - sbA) : 0;
    const uint32_t sb0 = min(sbA, p.sb_total - 1);
    constexpr uint32_t kMetaLive = 1u << 16, kMetaTileEnd = 1u << 17;
    uint32_t tw_lo, tw_hi, ts_lo = 0, ts_hi = 0, tmeta;
    // Segment si's scale array as segment 0's plus a difference chosen per
    // lane: a per-lane choice among the three pointers compiles to an
    // indexed load from a scratch copy of the argument block.
    static_assert(kFusedMaxSegs == 3, "one scale pointer per segment");
    const float* const tsc0 = uniform_ptr(p.seg[0].tscales);
    const int64_t tsc_d1 = uniform_ptr(p.seg[1].tscales) - tsc0;
    const int64_t tsc_d2 = uniform_ptr(p.seg[2].tscales) - tsc0;
    // the first superblock of tile `tile` of this slice, in a segment's
    // tile-ordered arrays
    auto tile_sb = [&](uint32_t tile) -> uint64_t {
        return static_cast<uint64_t>(tile) * (SLICED ? sb_stride : p.sb_total) + (SLICED ? ks * p.sb_total : 0u);
    };
    {
        const uint8_t* s_tiles[kFusedMaxSegs];
#pragma unroll
        for (uint32_t x = 0; x < kFusedMaxSegs; ++x) s_tiles[x] = uniform_ptr(p.seg[x].tiles);
        const uint32_t i = min(static_cast<uint32_t>(lane), items - 1);
        const uint32_t j = (i * p.len_magic) >> 16, q = i - j * len;
        uint32_t tile;
        const uint32_t si = seg_of(blockIdx.x + j * gridDim.x, tile);
        const uint64_t ts = tile_sb(tile) + sb0 + (q < nlive ? q : (nlive ? nlive - 1 : 0));
        const uint64_t w = reinterpret_cast<uint64_t>(SEG_PICK(s_tiles, si) + ts * SB_BYTES);
        tw_lo = static_cast<uint32_t>(w);
        tw_hi = static_cast<uint32_t>(w >> 32);
        if constexpr (!LS) {
            const float* const base = tsc0 + (si == 1 ? tsc_d1 : 0) + (si == 2 ? tsc_d2 : 0);
            const uint64_t sc = reinterpret_cast<uint64_t>(base + ts * 16 * gps);
            ts_lo = static_cast<uint32_t>(sc);
            ts_hi = static_cast<uint32_t>(sc >> 32);
        }
        tmeta = (q < nlive ? (sbA + q) | kMetaLive : 0u) | (q == len - 1 ? kMetaTileEnd : 0u);
    }
    // LS: the scales of the block's tiles, [tile j][segment slot][sb][16]
    // [gps] in LDS: each tile's run is contiguous in the tile-ordered scale
    // array, so the block loads them all at launch, ahead of the codes, at
    // most SC float4 per thread (the launch caps a block's tiles to fit):
    // per superblock the loop then issues one code load and reads its scale
    // from LDS.
    constexpr int SC = LS ? qgemv_scale_slots(NT, GPS, BITS) : 0;
    const uint32_t run4 = p.sb_total * 16 * gps / 4;  // float4 per tile and segment
    const uint32_t sc4_total = my_tiles * NT * run4;
    float4 scv[SC > 0 ? SC : 1];
    if constexpr (LS) {
        // float4 f of the block's runs is float4 o of run r = f / run4
        const uint32_t last = sc4_total ? sc4_total - 1 : 0;  // the launch gives every block a tile
        static_for<SC>([&](auto u_c) {
            constexpr int u = decltype(u_c)::value;
            const uint32_t f = min(static_cast<uint32_t>(tid + kThreads * u), last);
            const uint32_t r = __umulhi(f, p.run4_magic);
            const uint32_t o = f - r * run4;
            uint32_t tile = blockIdx.x + (r / NT) * gridDim.x;
            uint32_t si = r % NT;
            if (NT == 1) si = seg_of(tile, tile);
            const float* const base = tsc0 + (si == 1 ? tsc_d1 : 0) + (si == 2 ? tsc_d2 : 0);
            const v4f x = global_ptr(reinterpret_cast<const v4f*>(base + tile_sb(tile) * 16 * gps))[o];
            scv[u] = make_float4(x[0], x[1], x[2], x[3]);
        });
    }
    auto lane_u64 = [&](uint32_t lo, uint32_t hi, uint32_t k) {
        return static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(hi), k))) << 32 |
               static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lo), k));
    };
    auto fetch = [&](Item<BITS>& it, uint32_t k) {  // k wave-uniform
        k = min(k, items - 1);
        const auto wp = global_ptr(reinterpret_cast<const v4u*>(lane_u64(tw_lo, tw_hi, k))) + lane;
        const v4u w0 = wp[0];
        it.c0 = make_uint4(w0[0], w0[1], w0[2], w0[3]);
        if constexpr (BITS == 8) {
            const v4u w1 = wp[64];
            it.c1 = make_uint4(w1[0], w1[1], w1[2], w1[3]);
        }
        if constexpr (!LS) {
            const auto sp = global_ptr(reinterpret_cast<const float*>(lane_u64(ts_lo, ts_hi, k))) + (lane % 16) * gps;
            if constexpr (GPS == 2) {
                const v2f s2 = *reinterpret_cast<const __attribute__((address_space(1))) v2f*>(sp);
                it.s0 = s2[0];
                it.s1 = s2[1];
            } else {
                it.s0 = sp[0];
            }
        }
    };

    // Output element e of the block's [tiles][16][m] results: its segment
    // and offset, false past the segment's rows.
    auto out_at = [&](uint32_t e, uint32_t& si, uint64_t& o) -> bool {
        const uint32_t q = (e * p.m_magic) >> 16, j = q / 16, col = q % 16, m = e - q * M;
        uint32_t tile = blockIdx.x + j * gridDim.x;
        si = 0;
        if (NT == 1) si = seg_of(tile, tile);
        const uint32_t sn = SEG_PICK(s_n, si);
        const uint32_t orow = tile * 16 + col;
        o = static_cast<uint64_t>(m) * sn + orow;
        return orow < sn;
    };
    // The residual input of this thread's first output is loaded right
    // after the weight window, so the epilogue does not wait a memory round
    // trip for it. Every thread loads (threads without one re-read an
    // activation), which keeps the compiler's wait counts exact.
    const float* res_src = a_in;
    if (p.epilogue == kFusedResidual && static_cast<uint32_t>(tid) < my_tiles * 16 * M) {
        uint32_t si;
        uint64_t o;
        if (out_at(tid, si, o)) res_src = SEG_PICK(s_res, si) + o;
    }
    Item<BITS> win[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) fetch(win[i], i);
    const float res0 = *global_ptr(res_src);
    // a wave past the input (wave-uniform: whole runs) loaded the last run again
#pragma unroll
    for (int u = 0; u < F4; ++u)
        if (static_cast<uint32_t>(wave) * kWave + kThreads * u >= total4) v[u] = make_float4(0.f, 0.f, 0.f, 0.f);

    if (gamma != nullptr) {
        // each run's sum of squares over the wave: the F4 runs reduced
        // together, lane l ending with run l / (64 / F4)'s
        float ssq[F4];
#pragma unroll
        for (int u = 0; u < F4; ++u) {
            float ss = 0.f;
            ss = fmaf(v[u].x, v[u].x, ss);
            ss = fmaf(v[u].y, v[u].y, ss);
            ss = fmaf(v[u].z, v[u].z, ss);
            ss = fmaf(v[u].w, v[u].w, ss);
            ssq[u] = ss;
        }
        if constexpr (F4 == 1) {
            const float ss = wave_sum(ssq[0]);
            if (lane == 0) red[0][wave] = ss;
        } else {
            const float ss = lane_reduce_sum<F4>(ssq);
            if (lane % (kWave / F4) == 0) red[lane / (kWave / F4)][wave] = ss;
        }
        // Each wave sums the rows w, w + W over the (u, wave) partials of
        // their runs in a fixed order, and stores the row's 1 / rms.
        __syncthreads();
        const float kf = static_cast<float>(K);
        for (uint32_t r = wave; r < M; r += kWaves) {
            // kMaxF4 x W partials, one per lane for 8 waves, two for 16
            const uint32_t lo = r * K4, hi = lo + K4;
            float x = 0.f;
#pragma unroll
            for (int e0 = 0; e0 < kMaxF4 * kWaves; e0 += kWave) {
                const int e = e0 + lane, u = e / kWaves, w = e % kWaves;
                const uint32_t fb = static_cast<uint32_t>(w) * kWave + kThreads * u;
                if (fb < total4 && fb >= lo && fb < hi) x = e0 == 0 ? red[u][w] : x + red[u][w];
            }
            x = wave_sum(x);
            if (lane == 0) row_val[r] = 1.0f / sqrtf(x / kf + p.eps);
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < F4; ++u) {
            const uint32_t f = tid + kThreads * u;
            if (f < total4) {
                const float inv = row_val[ru[u]];
                const float4 g = gv[u];
                v[u].x = (v[u].x * inv) * g.x;
                v[u].y = (v[u].y * inv) * g.y;
                v[u].z = (v[u].z * inv) * g.z;
                v[u].w = (v[u].w * inv) * g.w;
                if (blockIdx.x == 0 && p.normed != nullptr) reinterpret_cast<float4*>(p.normed)[f] = v[u];
            }
        }
    }
    // Exact integers X = rint(x * 2^(22-E)) as three signed int8 limbs, with
    // E the exponent of the largest |x| of each 256-element chunk (one wave's
    // run): the wave that converts a chunk finds its maximum with a DPP
    // reduction, so no block-wide pass is needed. The integer sums are
    // combined per unit of min(group, 256) elements, which never spans two
    // chunks, each with its chunk's factor 2^(E-22) (2^(E-26) for INT4,
    // whose operands are the signed bytes 16 q).
    const uint32_t chunks = K / 256;
    int8_t* const limb_lane = limbs + 4 * lane;  // this lane's word of a limb row's run
    // max|x| of each run's chunk as a bit pattern (non-negative floats order
    // as unsigned integers): the F4 runs reduced together, lane l ending
    // with run l / (64 / F4)'s (F4 > 1)
    uint32_t lmax[F4];
#pragma unroll
    for (int u = 0; u < F4; ++u)
        lmax[u] = __float_as_uint(fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
    uint32_t rmax;
    if constexpr (F4 == 1) rmax = wave_max_u32(lmax[0]);
    else rmax = lane_reduce_max_u32<F4>(lmax);
#pragma unroll
    for (int u = 0; u < F4; ++u) {
        const uint32_t fb = static_cast<uint32_t>(wave) * kWave + kThreads * u;
        if (fb >= total4) continue;  // whole wave past the end
        const uint32_t r = ru[u];
        // ex = the chunk maximum's biased exponent - 126: frexp's exponent,
        // max|x| < 2^ex. A zero or subnormal maximum gives -126: the chunk's
        // X are then its values in units of 2^-148 (|X| < 2^22), which drops
        // at most the last bit of a subnormal, and its factor 2^(ex-22) is
        // itself subnormal (zero for INT4).
        const uint32_t mb = F4 == 1 ? rmax
                                    : static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(rmax),
                                                                                      u * (kWave / F4)));
        const int ex = static_cast<int>(mb >> 23) - 126;
        const int shift = 22 - ex;
        if (lane == 0) cfac[r * chunks + cb[u] / 64] = ldexpf(1.0f, ex - 22 - (BITS == 4 ? 4 : 0));
        // X from one fma: with |x * 2^shift| <= 2^22, y = x * 2^shift +
        // 1.5 * 2^23 rounds to an integer (ties to even, as rintf) and
        // bits(y) = 0x4B400000 + X. X + 0x808080 lies in [0, 2^24) and its
        // bytes b_i satisfy X = sum (b_i - 128) 256^i; v_perm gathers byte i
        // of the four elements into limb word i, and flipping the top bit
        // of every byte of a limb word makes its bytes the signed limbs. A
        // chunk whose 2^shift is not a normal float (max|x| < 2^-105)
        // scales in two exact steps.
        const float xe[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        uint32_t y[4];
        if (shift <= 127) {  // wave-uniform
            const float s2 = __uint_as_float(static_cast<uint32_t>(shift + 127) << 23);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                y[e] = __float_as_uint(fmaf(xe[e], s2, 12582912.0f)) - 0x4ABF7F80u;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float xs = xe[e] * 0x1p127f;  // exact: |x| < 2^-105
                y[e] = __float_as_uint(fmaf(xs, ldexpf(1.0f, shift - 127), 12582912.0f)) - 0x4ABF7F80u;
            }
        }
        const uint32_t lo01 = __builtin_amdgcn_perm(y[1], y[0], 0x05010400u);  // y0.b0 y1.b0 y0.b1 y1.b1
        const uint32_t lo23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010400u);
        const uint32_t hi01 = __builtin_amdgcn_perm(y[1], y[0], 0x07030602u);  // y0.b2 y1.b2 ..
        const uint32_t hi23 = __builtin_amdgcn_perm(y[3], y[2], 0x07030602u);
        const uint32_t packed[3] = {__builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u,
                                    __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u,
                                    __builtin_amdgcn_perm(hi23, hi01, 0x05040100u) ^ 0x80808080u};
#pragma unroll
        for (int limb = 0; limb < 3; ++limb)  // row limb * M + r, columns 4 cb[u] + 4 lane
            *reinterpret_cast<uint32_t*>(limb_lane + ((limb * M + r) * RS + 4 * cb[u])) = packed[limb];
    }
    static_for<SC>([&](auto u_c) {
        constexpr int u = decltype(u_c)::value;
        const uint32_t f = tid + kThreads * u;
        if (f < sc4_total) reinterpret_cast<float4*>(tsc)[f] = scv[u];
    });
    __syncthreads();

    // ---- main loop over the stream ----
    const uint32_t kb4 = lane / 16;
    // A-operand row of this lane: with LR row 4 * m + limb (limb 3 repeats
    // limb 2), else row m of each limb matrix; rows past M repeat row M - 1.
    // Their products are never read.
    uint32_t a_off;
    if constexpr (LR) {
        const uint32_t row = static_cast<uint32_t>(lane % 16);
        a_off = (min(row % 4, 2u) * M + min(row / 4, M - 1)) * RS;
    } else {
        a_off = min(static_cast<uint32_t>(lane % 16), M - 1) * RS;
    }
    constexpr int NR = LR ? 1 : 4;  // output rows a lane finishes (LR: m = kb4)
    const uint32_t steps_per_unit = p.unit / 64;
    const v4i zero = {0, 0, 0, 0};
    float total[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) total[r] = 0.f;
    // integer sums of the current group (a group may span superblocks; the
    // wave runs are group-aligned, so a group never spans two runs)
    v4i acc0 = zero, acc1 = zero, acc2 = zero;
    uint32_t cj = 0;                      // block tile of the item being consumed
    // this lane's scales: row lane % 16 of its segment slot, tile cj
    const float* const tsc_lane = tsc + slot * p.sb_total * 16 * gps + (lane % 16) * gps;
    const uint32_t tile_stride = NT * p.sb_total * 16 * gps;
    uint32_t gstep = 0;                   // 64-k steps into the current unit
    const int8_t* a_col = limbs + a_off + kb4 * 16;
    // One item of the stream: win[S] is used in place (a copy would make the
    // compiler wait before its refill) and refilled afterwards. A dead item
    // (a trailing wave's padding past k) computes on clamped addresses and
    // its sums are dropped by a select rather than a branch.
    auto consume = [&](auto s_c, uint32_t meta) {
        constexpr int S = decltype(s_c)::value;
        const Item<BITS>& cur = win[S];
        const bool use = (meta & kMetaLive) != 0;
        const uint32_t sbi = meta & 0xffffu;  // superblock along k (dead: 0)
        const int8_t* ap = a_col + sbi * 128;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            v4i bv;
            if (BITS == 4) {
                const uint32_t wa = st == 0 ? cur.c0.x : cur.c0.z;
                const uint32_t wb = st == 0 ? cur.c0.y : cur.c0.w;
                // two's complement nibbles -> the signed bytes 16 q
                bv[0] = static_cast<int>((wa << 4) & 0xF0F0F0F0u);
                bv[1] = static_cast<int>(wa & 0xF0F0F0F0u);
                bv[2] = static_cast<int>((wb << 4) & 0xF0F0F0F0u);
                bv[3] = static_cast<int>(wb & 0xF0F0F0F0u);
            } else {
                const uint4 cw = st == 0 ? cur.c0 : cur.c1;
                bv[0] = static_cast<int>(cw.x);
                bv[1] = static_cast<int>(cw.y);
                bv[2] = static_cast<int>(cw.z);
                bv[3] = static_cast<int>(cw.w);
            }
            if constexpr (LR) {
                // a group's first step starts from zero (no reset moves)
                const bool fresh = SPG == 1 || (SPG == 2 && st == 0);
                const v4i a0 = *reinterpret_cast<const v4i*>(ap + st * 64);
                acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bv, fresh ? zero : acc0, 0, 0, 0);
            } else {
                const v4i a0 = *reinterpret_cast<const v4i*>(ap + st * 64);
                const v4i a1 = *reinterpret_cast<const v4i*>(ap + M * RS + st * 64);
                const v4i a2 = *reinterpret_cast<const v4i*>(ap + 2 * M * RS + st * 64);
                acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bv, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bv, acc1, 0, 0, 0);
                acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, bv, acc2, 0, 0, 0);
            }
            bool group_end;
            if constexpr (SPG == 1) group_end = true;
            else if constexpr (SPG == 2) group_end = st == 1;
            else group_end = ++gstep == steps_per_unit;
            if (group_end) {
                if constexpr (SPG == 0) gstep = 0;
                float sc;
                if constexpr (LS) sc = tsc_lane[cj * tile_stride + sbi * 16 * gps + (GPS == 2 && st == 1 ? 1 : 0)];
                else sc = GPS == 2 && st == 1 ? cur.s1 : cur.s0;
                const uint32_t chunk = (sbi * 128 + st * 64) / 256;
                if constexpr (LR) {
                    // rows 4 * kb4 + limb: this lane holds all three limbs of m = kb4
                    const uint32_t m = min(kb4, M - 1);
                    float val = fmaf(static_cast<float>(acc0[2]), 65536.0f,
                                     fmaf(static_cast<float>(acc0[1]), 256.0f, static_cast<float>(acc0[0])));
                    const float t = fmaf(val * cfac[m * chunks + chunk], sc, total[0]);
                    total[0] = use ? t : total[0];
                } else {
#pragma unroll
                    for (int r = 0; r < NR; ++r) {
                        const uint32_t m = min(kb4 * 4 + r, M - 1);
                        float val = fmaf(static_cast<float>(acc2[r]), 65536.0f,
                                         fmaf(static_cast<float>(acc1[r]), 256.0f, static_cast<float>(acc0[r])));
                        const float t = fmaf(val * cfac[m * chunks + chunk], sc, total[r]);
                        total[r] = use ? t : total[r];
                    }
                }
                acc0 = zero;
                acc1 = zero;
                acc2 = zero;
            }
        }
    };
    // tile j done: wave partials -> LDS, summed in wave order into the
    // block's result area (global writes wait until the stream is done, so
    // the loop issues only the window's loads)
    auto tile_end = [&]() {
        const uint32_t j = cj;
        ++cj;
        const uint32_t buf = j & 1;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            wres[buf][wave][LR ? kb4 : kb4 * 4 + r][lane % 16] = total[r];
            total[r] = 0.f;
        }
        __syncthreads();
        if (static_cast<uint32_t>(tid) < 16 * M) {
            const uint32_t m = tid / 16, col = tid % 16;
            float val;
            if (NT == 1) {
                float acc = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) acc += wres[buf][w][m][col];
                val = acc;
            } else {
                float g = 0.f, up = 0.f;
#pragma unroll
                for (int w = 0; w < WPT; ++w) {
                    g += wres[buf][w][m][col];
                    up += wres[buf][WPT + w][m][col];
                }
                val = (g * (1.0f / (1.0f + expf(-g)))) * up;
            }
            tres[(j * 16 + col) * M + m] = val;
        }
    };
    // Rounds of PF items; in the last one the items past the stream do no
    // work and no tile bookkeeping but still refill their slot (with the
    // last item again). There is no exit inside a round, so every wait stays
    // one item deep: an early exit, or a second copy of the round for the
    // tail, makes the compiler wait for the whole window.
    for (uint32_t base = 0; base < items; base += PF) {
        static_for<PF>([&](auto s_c) {
            const uint32_t k = base + decltype(s_c)::value;
            const bool live = k < items;
            const uint32_t meta = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(tmeta), min(k, items - 1)));
            if (live) consume(s_c, meta);
            if constexpr (SM != kSmOneRound) fetch(win[decltype(s_c)::value], k + PF);
            if (live && (meta & kMetaTileEnd)) tile_end();
        });
    }

    // ---- results of all the block's tiles ----
    __syncthreads();
    for (uint32_t e = tid; e < my_tiles * 16 * M; e += kThreads) {
        uint32_t si;
        uint64_t o;
        if (!out_at(e, si, o)) continue;
        const float val = tres[e];
        global_ptr(SEG_PICK(s_out, si))[o] = val;
        if (p.epilogue == kFusedResidual)
            global_ptr(SEG_PICK(s_out2, si))[o] = (e == tid ? res0 : global_ptr(SEG_PICK(s_res, si))[o]) + val;
    }
}
#undef SEG_PICK

// out[i] = the sum of the k slices' partials of element i, in slice order;
// with resid, out2[i] = resid[i] + out[i] (the residual Add's order).
__global__ __launch_bounds__(256) void qgemv_slices_sum(const float* __restrict__ partial, uint32_t slices,
                                                        uint64_t count, float* out, const float* resid,
                                                        float* out2) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += static_cast<uint64_t>(gridDim.x) * 256) {
        float v = partial[i];
        for (uint32_t sl = 1; sl < slices; ++sl) v += partial[sl * count + i];
        out[i] = v;
        if (out2 != nullptr) out2[i] = resid[i] + v;
    }
}

}  // namespace

hipError_t launch_qgemv_fused(const QgemvFused& f, hipStream_t s) {
    if (f.nseg == 0 || f.nseg > kFusedMaxSegs || f.m == 0 || f.m > 16) return hipErrorNotSupported;
    const QuantWeight& w0 = *f.w[0];
    const uint64_t k = w0.k;
    if (w0.layout != QuantLayout::Mfma || k % 256 != 0 || w0.group % 64 != 0 || k % w0.group != 0 ||
        !(w0.group == 64 || w0.group == 128 || w0.group % 256 == 0) || !aligned16(f.a) ||
        (f.gamma != nullptr && !aligned16(f.gamma)) || (f.normed != nullptr && !aligned16(f.normed)))
        return hipErrorNotSupported;
    if (f.epilogue == kFusedPair && f.nseg != 2) return hipErrorNotSupported;
    // Activations beyond the LDS (m x k above max_elems(16): the down
    // projection, k = 14336, at batch 8): the grid's y dimension cuts k into
    // slices that fit, each block converting only its slice; the slices'
    // partial sums go to f.partial and a second launch adds them up (and
    // the residual). Single weights without a norm prologue only.
    uint32_t slices = 1;
    if (f.m * k > max_elems(16)) {
        if (f.gamma != nullptr || f.epilogue == kFusedPair || f.nseg != 1 || f.partial == nullptr)
            return hipErrorNotSupported;
        const uint64_t unit = w0.group > 256 ? w0.group : 256;
        while (slices <= 16 && (k % (slices * unit) != 0 || f.m * (k / slices) > max_elems(16))) ++slices;
        if (slices > 16 || slices * f.m * w0.n > f.partial_floats) return hipErrorNotSupported;
    }
    const uint64_t kc = k / slices;
    Args p;
    p.normed = f.normed;
    p.eps = f.eps;
    p.nseg = f.nseg;
    p.m = static_cast<uint32_t>(f.m);
    p.k = static_cast<uint32_t>(kc);
    p.group = w0.group;
    p.sb_total = p.k / 128;
    p.groups_total = p.k / p.group;
    p.unit = p.group < 256 ? p.group : 256;
    p.epilogue = slices > 1 ? kFusedPlain : f.epilogue;
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < f.nseg; ++i) {
        const QuantWeight& w = *f.w[i];
        if (w.layout != QuantLayout::Mfma || w.tile_scales == nullptr || w.k != k || w.group != w0.group ||
            w.format != w0.format || w.n > 0xffffffffull)
            return hipErrorNotSupported;
        if (f.epilogue == kFusedPair && w.n != w0.n) return hipErrorNotSupported;
        p.seg[i] = Seg{w.tiles, w.tile_scales, slices > 1 ? f.partial : f.out[i], f.resid[i], f.out2[i],
                       static_cast<uint32_t>(w.n), tiles};
        if (f.epilogue != kFusedPair) tiles += static_cast<uint32_t>((w.n + 15) / 16);
    }
    if (f.epilogue == kFusedPair) tiles = static_cast<uint32_t>((w0.n + 15) / 16);
    p.tiles_total = tiles;
    const bool int4 = w0.format == SL_QFORMAT_INT4, pair = f.epilogue == kFusedPair, lr = p.m <= 4;
    // Waves per block: 16 for long k (the down projection, k = 14336), which
    // doubles the weight loads in flight per CU and halves each thread's
    // share of the activation prologue, and for a single weight above 24 MB
    // whose tiles one round of 16-wave blocks holds (one block per CU
    // instead of two converting the same activations): [14336 x 4096] 7.95-
    // 8.04 -> 7.74-7.83 us. 8 otherwise: with 16, lm_head [128256 x 4096]
    // 47.0 -> 48.1 us, q/k/v and o-proj [4096 x 4096] 0.8 us slower together.
    const uint64_t weight_bytes = static_cast<uint64_t>(tiles) * p.sb_total * (int4 ? 1024 : 2048) * (pair ? 2 : 1);
    const bool wide = !pair && p.m == 1 && p.k >= 4096 && weight_bytes > (24ull << 20) &&
                      tiles <= 4 * compute_units();
    const int waves = p.k >= 8192 || p.m * p.k > max_elems(8) || wide ? 16 : 8;
    const uint32_t threads = static_cast<uint32_t>(waves) * kWave;
    const uint32_t wpt = f.epilogue == kFusedPair ? waves / 2 : waves;
    const uint32_t sb_per_group = p.group >= 128 ? p.group / 128 : 1;
    uint32_t per = (p.sb_total + wpt - 1) / wpt;
    per = (per + sb_per_group - 1) / sb_per_group * sb_per_group;
    p.sb_per_wave = per;
    // Resident blocks: every block converts the activations once for all
    // its tiles; the results of a block's tiles wait in LDS (at most 16 KB).
    // Weights of up to 24 MB take one block per CU, the tiles dealt round
    // robin (some blocks one more): the prologue, repeated by every block,
    // is then paid once per CU. Larger ones take up to two per CU, with
    // even shares, for more loads in flight. (Measured on MI355X, M = 1:
    // the q/k/v launch [6144 x 4096] gains 1 us from one block per CU, the
    // gate/up pair [2 x 14336 x 4096] loses 0.5 us.)
    uint32_t blocks, per_block;
    const uint32_t per_cap = 4096 / (16 * p.m);
    if (slices > 1) {
        // about one block per CU over all slices: each block converts its
        // slice's activations once for several tiles
        blocks = (compute_units() + slices - 1) / slices;
        if (blocks > tiles) blocks = tiles;
        per_block = (tiles + blocks - 1) / blocks;
    } else if (weight_bytes <= (24ull << 20)) {
        blocks = tiles < compute_units() ? tiles : compute_units();
        per_block = (tiles + blocks - 1) / blocks;
    } else {
        const uint32_t max_blocks = (waves == 16 ? 1 : 2) * compute_units();
        per_block = (tiles + max_blocks - 1) / max_blocks;
        blocks = 0;
    }
    // Float4 of activations per thread, a compile-time count: the prologue
    // is straight-line code run once per wave, fetched cold by every CU at
    // each launch, so its length shows in the launch time (about 1 us for
    // the RMSNorm prologue at 8 float4 per thread against 2).
    const uint32_t f4 = (p.m * p.k / 4 + threads - 1) / threads;
    // Scales in LDS (LS) for one activation row, k >= 4096 and more
    // superblocks per wave than the window holds. Measured on MI355X
    // against scales loaded with each superblock: [14336 x 4096] 8.61 ->
    // 8.45 us, [4096 x 14336] 9.24 -> 9.00 us, the gate/up pair [2 x 14336
    // x 4096] 13.62 -> 13.32 us; but [2048 x 8192] (4 superblocks per
    // wave) 5.80 -> 6.34 us, and M = 8 [14336 x 4096] 13.73 -> 14.38 us.
    const bool ls = p.m == 1 && slices == 1 && p.k >= 4096 && f4 <= 4 && per_block * per > kWindow;
    // A stream that fits the first window (every block's tiles times the
    // superblocks per wave; the cap below only lowers per_block) is one
    // round without refills: [2048 x 8192] 5.50 -> 5.20 us, [2048 x 2048]
    // 3.77 -> 3.60 us. Dropping the refills of a longer stream's last round
    // instead makes the compiler's waits cover more than one item:
    // [14336 x 4096] 8.45 -> 8.69 us.
    const bool one_round = !ls && lr && slices == 1 && f4 <= 4 && per_block * per <= kWindow;
    // the per-lane item table holds at most 64 items per wave, and with LS
    // the tiles' scales at most qgemv_scale_slots float4 per thread
    const uint32_t gps = p.group == 64 ? 2 : 1, nt = pair ? 2 : 1;
    uint32_t item_cap = 64 / per;
    if (ls) {
        const uint32_t scale_cap =
            static_cast<uint32_t>(qgemv_scale_slots(nt, gps, int4 ? 4 : 8)) * threads / (nt * p.sb_total * 4 * gps);
        if (scale_cap < item_cap) item_cap = scale_cap;
    }
    const uint32_t cap = per_cap < item_cap ? per_cap : item_cap;
    if (cap == 0) return hipErrorNotSupported;
    if (per_block > cap) per_block = cap;
    if (blocks == 0 || per_block == cap) blocks = (tiles + per_block - 1) / per_block;
    p.tile_slots = per_block;
    p.tiles_base = tiles / blocks;
    p.tiles_rem = tiles % blocks;
    p.len_magic = magic16(per);
    p.m_magic = magic16(p.m);
    p.run4_magic = static_cast<uint32_t>(((1ull << 32) + run4_of(p.sb_total, gps) - 1) / run4_of(p.sb_total, gps));
    const uint32_t mk = p.m | (magic16(p.k / 256) << 5);
    const size_t lds = static_cast<size_t>(3) * p.m * (p.k + kLimbPad) +
                       sizeof(float) * static_cast<size_t>(per_block) * 16 * p.m +
                       (ls ? sizeof(float) * static_cast<size_t>(per_block) * nt * p.sb_total * 16 * gps : 0);
    if (lds + static_lds(waves) > max_lds_per_block()) return hipErrorNotSupported;
    const int spg = p.group == 64 ? 1 : p.group == 128 ? 2 : 0;
    const dim3 grid(blocks, slices);
#define SL_QGEMV_LAUNCH(B, T, G, L, F, W, S) \
    qgemv_fused<B, T, G, L, F, W, false, S><<<grid, threads, lds, s>>>(f.a, f.gamma, mk, p.k, p)
#define SL_QGEMV_FUSED_F(B, T, G, L)                                                                               \
    (waves == 16 ? (f4 <= 2 ? SL_QGEMV_LAUNCH(B, T, G, L, 2, 16, kSmStream)                                             \
                            : f4 <= 4 ? SL_QGEMV_LAUNCH(B, T, G, L, 4, 16, kSmStream) : SL_QGEMV_LAUNCH(B, T, G, L, 8, 16, kSmStream)) \
                 : f4 <= 2 ? SL_QGEMV_LAUNCH(B, T, G, L, 2, 8, kSmStream)                                               \
                           : f4 <= 4 ? SL_QGEMV_LAUNCH(B, T, G, L, 4, 8, kSmStream) : SL_QGEMV_LAUNCH(B, T, G, L, 8, 8, kSmStream))
#define SL_QGEMV_FUSED_SM(B, T, G, S)                                                                               \
    (waves == 16 ? (f4 <= 2 ? SL_QGEMV_LAUNCH(B, T, G, true, 2, 16, S) : SL_QGEMV_LAUNCH(B, T, G, true, 4, 16, S)) \
                 : f4 <= 2 ? SL_QGEMV_LAUNCH(B, T, G, true, 2, 8, S) : SL_QGEMV_LAUNCH(B, T, G, true, 4, 8, S))
#define SL_QGEMV_FUSED(B, T, G) \
    (ls ? SL_QGEMV_FUSED_SM(B, T, G, kSmLds)                                          \
        : one_round ? SL_QGEMV_FUSED_SM(B, T, G, kSmOneRound)                         \
                    : lr ? SL_QGEMV_FUSED_F(B, T, G, true) : SL_QGEMV_FUSED_F(B, T, G, false))
#define SL_QGEMV_FUSED_G(B, T) \
    (spg == 1 ? SL_QGEMV_FUSED(B, T, 1) : spg == 2 ? SL_QGEMV_FUSED(B, T, 2) : SL_QGEMV_FUSED(B, T, 0))
    if (slices > 1) {
        // k slices: many rows (not LR), 16 waves, 8 float4 per thread
        if (waves != 16 || f4 > 8 || lr) return hipErrorNotSupported;
#define SL_QGEMV_SLICED(B, G) qgemv_fused<B, 1, G, false, 8, 16, true, kSmStream><<<grid, threads, lds, s>>>(f.a, f.gamma, mk, p.k, p)
        if (int4) {
            if (spg == 1) SL_QGEMV_SLICED(4, 1);
            else if (spg == 2) SL_QGEMV_SLICED(4, 2);
            else SL_QGEMV_SLICED(4, 0);
        } else {
            if (spg == 1) SL_QGEMV_SLICED(8, 1);
            else if (spg == 2) SL_QGEMV_SLICED(8, 2);
            else SL_QGEMV_SLICED(8, 0);
        }
#undef SL_QGEMV_SLICED
    } else if (int4) {
        if (pair) SL_QGEMV_FUSED_G(4, 2);
        else SL_QGEMV_FUSED_G(4, 1);
    } else {
        if (pair) SL_QGEMV_FUSED_G(8, 2);
        else SL_QGEMV_FUSED_G(8, 1);
    }
#undef SL_QGEMV_FUSED_G
#undef SL_QGEMV_FUSED
#undef SL_QGEMV_FUSED_SM
#undef SL_QGEMV_FUSED_F
#undef SL_QGEMV_LAUNCH
    if (slices > 1) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const uint64_t count = f.m * w0.n;
        const bool residual = f.epilogue == kFusedResidual;
        qgemv_slices_sum<<<grid_for(count, 256, 1024), 256, 0, s>>>(f.partial, slices, count, f.out[0],
                                                                   residual ? f.resid[0] : nullptr,
                                                                   residual ? f.out2[0] : nullptr);
    }
    return hipGetLastError();
}

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_qgemv_fused() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&qgemv_slices_sum));
}

}  // namespace slhip
