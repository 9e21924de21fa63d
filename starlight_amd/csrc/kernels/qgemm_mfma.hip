// Group-quantized MatMulNT for many activation rows (prefill):
// out[m, n] = sum_k a[m, k] * (q[n, k] * s[n, k / G]), on the fp16 matrix
// cores, from the Mfma tile layout of the weights.
//
// Exactness plan. The codes q are small integers, exact in fp16. Each
// activation row is scaled by 2^(15 - E) (|a| < 2^E over the row, so the
// scaled values stay below the fp16 maximum) and split into a high and a
// low fp16 part, a' = hi + lo, which keeps about 22 significant bits of
// every element (elements far below the row maximum keep an absolute error
// below 2^-25 of it). v_mfma_f32_16x16x32_f16 forms hi * q and lo * q exactly
// and sums them in f32 over one quantization group; the group's sum is then
// multiplied by its scale and added to the f32 result, and the result is
// scaled back by 2^(E - 15). Against matmul_nt(a, dequant(q, s))
// (reference/matmul.rs:29-59, dequant one f32 multiply q * s) the only
// differences are f32 rounding (summation order, the scale applied per
// group instead of per weight) and the split's 2^-22: about 1e-6 normwise,
// inside the 1e-4 bound.
//
// Kernels
//  * split_rows: one block per row: E, then hi/lo in fp16 ([m][k] each,
//    every group of 8 along k in the order kPerm8) and E per row into the
//    workspace;
//  * qgemm_mfma: 128 x 128 output tiles, 4 waves of 64 x 64 (4 x 4 MFMA
//    tiles of 16 x 16), k in stages of 32 through double-buffered LDS; or
//    64 x 128 tiles (waves of 32 x 64) in stages of 32 or 64; a grid z of
//    2 cuts k in two slices whose partial sums gemm_slices_sum adds. The
//    weight stage is read from the tile layout (per 16-row tile and 128-k
//    superblock; a 32-k stage is half of one 64-k half: 32 lanes x 8 bytes
//    for INT4, x 16 bytes for INT8) and converted to fp16 codes in LDS
//    (codes8: through the mantissa of 1024, no converts).
#include "common.h"
#include "kernels.h"
#include "starlight_hip.h"

#include <type_traits>

namespace slhip {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kTile = 128;     // output columns per block (rows: BM, 128 or 64)
constexpr int kStepK = 32;     // k per MFMA step (an LDS stage holds KS = 32 or 64)
// halves per LDS row: 96 bytes for 32-k stages (80 and 112 measured
// slower); 144 bytes for 64-k stages, which puts the 16 rows one operand
// read spans on 16 disjoint groups of 4 banks
template <int KS>
constexpr int row_pad() { return KS == 32 ? 48 : 72; }
constexpr int kExpBias = 15;   // scaled rows stay below 2^15

// The activation element: a, or with a second input u (SwiGlu's down
// projection) silu(a) * u, the elementwise kernels' formula
// (elementwise.rs:10-12): (a * (1 / (1 + exp(-a)))) * u.
__device__ __forceinline__ float4 act4(const float4* row, const float4* urow, uint32_t i) {
    float4 v = row[i];
    if (urow != nullptr) {
        const float4 u = urow[i];
        v.x = (v.x * (1.0f / (1.0f + expf(-v.x)))) * u.x;
        v.y = (v.y * (1.0f / (1.0f + expf(-v.y)))) * u.y;
        v.z = (v.z * (1.0f / (1.0f + expf(-v.z)))) * u.z;
        v.w = (v.w * (1.0f / (1.0f + expf(-v.w)))) * u.w;
    }
    return v;
}

// Within every aligned group of 8 along k, position j of the split
// activations and of the converted codes holds element kPerm8[j]: the order
// in which the code conversion below takes nibble (and byte) pairs out of
// a word. Both operands share it, so the products pair up as before.
__device__ constexpr int kPerm8[8] = {0, 2, 4, 6, 1, 3, 5, 7};

// Row r: E with max |a| < 2^E (0 for an all-zero row), then hi/lo of
// a * 2^(15 - E); with u, of silu(a) * u; with gamma (NP > 0, k <= 8192,
// no u), of RMSNorm(a) * gamma. k % 8 == 0 and rows 16-byte aligned.
// NP > 0: the row's values stay in registers between the two passes
// (thread t holds the 8-element groups t + 256 j, j < NP, so k <= 2048 NP),
// and a and u are read once; NP == 0 reads the row twice.
template <int NP>
__global__ __launch_bounds__(256) void split_rows(const float* __restrict__ a, const float* __restrict__ u,
                                                  _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                  int* __restrict__ row_exp, uint32_t k,
                                                  const float* __restrict__ gamma, float eps) {
    __shared__ float scratch[4];
    const uint64_t r = blockIdx.x;
    const float4* row = reinterpret_cast<const float4*>(a + r * k);
    const float4* urow = u != nullptr ? reinterpret_cast<const float4*>(u + r * k) : nullptr;
    const uint32_t k4 = k / 4;
    const uint32_t groups = k4 / 2;  // eight elements each
    float4 keep[NP > 0 ? 2 * NP : 1];
    float mx = 0.f;
    if constexpr (NP > 0) {
        if (gamma != nullptr) {
            // RMSNorm first. Its sum of squares runs in the standalone
            // kernel's order (rms_norm_vec: thread t over float4 columns t +
            // 256 i, ascending, then block_sum), from a second set of loads
            // of the row, so the normalised values are bit-identical to that
            // kernel's output. Every load is unconditional (clamped indices;
            // columns past the row count as zeros, which leave the sum
            // unchanged) and issued before any of them is used.
            const float4* g4 = reinterpret_cast<const float4*>(gamma);
            float4 xv[2 * NP], gv[2 * NP];
#pragma unroll
            for (int j = 0; j < NP; ++j) {
                const uint32_t i = min(threadIdx.x + 256u * j, groups - 1);
                keep[2 * j] = row[2 * i];
                keep[2 * j + 1] = row[2 * i + 1];
                gv[2 * j] = g4[2 * i];
                gv[2 * j + 1] = g4[2 * i + 1];
            }
#pragma unroll
            for (int i = 0; i < 2 * NP; ++i) xv[i] = row[min(threadIdx.x + 256u * i, k4 - 1)];
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 2 * NP; ++i) {
                const float4 v = threadIdx.x + 256u * i < k4 ? xv[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                ss = fmaf(v.x, v.x, ss);
                ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss);
                ss = fmaf(v.w, v.w, ss);
            }
            ss = block_sum(ss, scratch);
            const float inv = 1.0f / sqrtf(ss / static_cast<float>(k) + eps);
#pragma unroll
            for (int j = 0; j < 2 * NP; ++j) {
                float4& v = keep[j];
                v.x = (v.x * inv) * gv[j].x;
                v.y = (v.y * inv) * gv[j].y;
                v.z = (v.z * inv) * gv[j].z;
                v.w = (v.w * inv) * gv[j].w;
                // groups past the row repeat the last one: the maximum is unchanged
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
        } else {
#pragma unroll
            for (int j = 0; j < NP; ++j) {
                const uint32_t i = threadIdx.x + 256 * j;
                if (i < groups) {
                    keep[2 * j] = act4(row, urow, 2 * i);
                    keep[2 * j + 1] = act4(row, urow, 2 * i + 1);
                    const float4 v0 = keep[2 * j], v1 = keep[2 * j + 1];
                    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))));
                    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
                }
            }
        }
    } else {
        for (uint32_t i = threadIdx.x; i < k4; i += 256) {
            const float4 v = act4(row, urow, i);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    }
    mx = block_max(mx, scratch);
    int e = 0;
    if (mx != 0.f) frexpf(mx, &e);  // mx < 2^e
    if (threadIdx.x == 0) row_exp[r] = e;
    const int shift = kExpBias - e;
    // eight elements per step, stored in the order kPerm8 (the order the
    // weight conversion produces codes in)
    auto put8 = [&](uint32_t i, float4 v0, float4 v1) {
        const float x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        v8h h, l;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float xs = ldexpf(x[kPerm8[j]], shift);
            h[j] = static_cast<_Float16>(xs);
            l[j] = static_cast<_Float16>(xs - static_cast<float>(h[j]));  // the subtraction is exact
        }
        *reinterpret_cast<v8h*>(hi + r * k + 8 * i) = h;
        *reinterpret_cast<v8h*>(lo + r * k + 8 * i) = l;
    };
    if constexpr (NP > 0) {
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            const uint32_t i = threadIdx.x + 256 * j;
            if (i < groups) put8(i, keep[2 * j], keep[2 * j + 1]);
        }
    } else {
        for (uint32_t i = threadIdx.x; i < groups; i += 256) put8(i, act4(row, urow, 2 * i), act4(row, urow, 2 * i + 1));
    }
}

// out[i] = the k slices' partial sums of element i, added in slice order;
// with resid, out2[i] = resid[i] + out[i] (the residual Add's order), and
// out may then be null (the sum itself not written).
__global__ __launch_bounds__(256) void gemm_slices_sum(const float* __restrict__ partial, uint32_t slices,
                                                       uint64_t count, float* out, const float* resid, float* out2) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += static_cast<uint64_t>(gridDim.x) * 256) {
        float v = partial[i];
        for (uint32_t z = 1; z < slices; ++z) v += partial[z * count + i];
        if (out != nullptr) out[i] = v;
        if (out2 != nullptr) out2[i] = resid[i] + v;
    }
}

// One stage's share of a thread: two 16-byte chunks of each of hi and lo,
// the weight bytes (INT4: the first 8), and the scale of column tid % 128
// for the stage's quantization group.
struct StageRegs {
    uint4 h0, l0, h1, l1, b, b2;  // b2: 64-k stages of INT8 weights
    float sc;
};

// One weight of a launch: its column blocks are block0 .. the next
// segment's block0 (up to three weights reading the same activations, such
// as q/k/v, run as one launch).
struct GemmSeg {
    const uint8_t* tiles;   // Mfma layout
    const float* scales;    // [n, k / group], row-major
    float* out;             // [m, n]
    const float* resid;     // with out2: out2 = resid + out (a residual Add), else null
    float* out2;
    uint32_t n, block0;
};

struct GemmArgs {
    const _Float16* ahi;
    const _Float16* alo;
    const int* row_exp;
    GemmSeg seg[kFusedMaxSegs];
    uint32_t nseg, m, k, group, groups, sb_total;
    // k cut into gridDim.z slices of k / gridDim.z (one weight only): slice z
    // writes its m x n partial sums at partial + z m n, added up afterwards
    float* partial;
};

typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Two codes held in the low bits of the two 16-bit halves of w (offset
// binary, code + bias, at most 8 bits) as fp16: OR-ing them into the
// mantissa of 1024 (0x6400) makes 1024 + code + bias exactly, and one packed
// subtraction leaves the code.
__device__ __forceinline__ uint32_t pair_f16(uint32_t w, uint32_t mask, float bias) {
    const uint32_t x = (w & mask) | 0x64006400u;
    v2h h = __builtin_bit_cast(v2h, x);
    const _Float16 b = static_cast<_Float16>(1024.0f + bias);
    h -= v2h{b, b};
    return __builtin_bit_cast(uint32_t, h);
}

// Eight signed codes as fp16 in the order kPerm8. INT4: one word, byte b
// holding codes b (low nibble) and 4 + b (high); flipping bit 3 of every
// nibble makes them offset binary (code + 8). INT8: two words (codes 0..3,
// 4..7), bit 7 flipped (code + 128).
template <int BITS>
__device__ __forceinline__ v8h codes8(uint32_t w0, uint32_t w1) {
    uint32_t d[4];
    if constexpr (BITS == 4) {
        const uint32_t x = w0 ^ 0x88888888u;
        d[0] = pair_f16(x, 0x000F000Fu, 8.f);        // codes 0, 2
        d[1] = pair_f16(x >> 4, 0x000F000Fu, 8.f);   // 4, 6
        d[2] = pair_f16(x >> 8, 0x000F000Fu, 8.f);   // 1, 3
        d[3] = pair_f16(x >> 12, 0x000F000Fu, 8.f);  // 5, 7
    } else {
        const uint32_t x = w0 ^ 0x80808080u, y = w1 ^ 0x80808080u;
        d[0] = pair_f16(x, 0x00FF00FFu, 128.f);       // codes 0, 2
        d[1] = pair_f16(y, 0x00FF00FFu, 128.f);       // 4, 6
        d[2] = pair_f16(x >> 8, 0x00FF00FFu, 128.f);  // 1, 3
        d[3] = pair_f16(y >> 8, 0x00FF00FFu, 128.f);  // 5, 7
    }
    return __builtin_bit_cast(v8h, d);
}

// GS: stages per quantization group known at compile time (4: 32-k stages,
// group 128; 2: 64-k stages and group 128, or 32-k stages and group 64), or
// 0 for any group (counted at run time).
template <int BITS, int BM, int KS, int GS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void qgemm_mfma(GemmArgs p) {
    static_assert(BM == 128 || BM == 64, "block rows");
    static_assert(KS == 32 || KS == 64, "stage depth");
    constexpr int CPR = KS / 8;  // 16-byte chunks per row and stage
    static_assert(BM * CPR <= 512, "at most two activation chunks per plane per thread");
    constexpr int MT = BM / 32;  // 16-row tiles per wave (a wave owns BM / 2 rows)
    constexpr int RP = row_pad<KS>();
    prefetch_kernarg<arg_bytes<GemmArgs>()>();
    __shared__ __align__(16) _Float16 as[2][2][BM][RP];      // [stage][hi, lo][row][k]
    __shared__ __align__(16) _Float16 bs[2][kTile][RP];     // [stage][column][k]
    __shared__ float ss[2][kTile];                           // [stage][column]: the group's scales
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const int wm = wave / 2, wn = wave % 2;
    // this block's weight, chosen with selects (block-uniform, in scalar
    // registers; a runtime index into the arguments would be a memory load)
    // this block's column block bx, row block by and k slice bz
    const uint32_t bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
    const uint32_t si = (p.nseg > 1 && bx >= p.seg[1].block0 ? 1u : 0u) + (p.nseg > 2 && bx >= p.seg[2].block0 ? 1u : 0u);
#define SL_GSEG(f) (si == 0 ? p.seg[0].f : si == 1 ? p.seg[1].f : p.seg[2].f)
    const uint8_t* const tiles = SL_GSEG(tiles);
    const float* const scales = SL_GSEG(scales);
    float* const out = SL_GSEG(out);
    const float* const resid = SL_GSEG(resid);
    float* const out2 = SL_GSEG(out2);
    const uint32_t n = SL_GSEG(n), n_tiles = (n + 15) / 16;
    const uint32_t m0 = by * BM, n0 = (bx - SL_GSEG(block0)) * kTile;
#undef SL_GSEG
    const uint32_t kslice = p.k / gridDim.z, kbeg = bz * kslice;  // this block's k range
    const uint32_t steps = kslice / KS, group_steps = p.group / KS;

    // This thread's share of a stage: one 16-byte chunk of each of hi and lo
    // per 256 / CPR rows of the block (row c / CPR, halves 8 (c % CPR) ..),
    // and of the weights (tile layout: per 16-row tile and 64-k half of a
    // superblock, lane L holds 16 codes of column L % 16, k 16 (L / 16) ..):
    // 32-k stages, lanes 32 t .. 32 t + 31 of tile tid / 32 (bi = tid % 32);
    // 64-k stages, lane tid % 64 of tiles tid / 64 and tid / 64 + 4.
    // (plain variables, not arrays: an array the lambdas capture would be
    // placed in LDS by the compiler)
    const uint32_t c0 = tid, c1 = tid + 256;
    const uint64_t aoff0 = static_cast<uint64_t>(min(m0 + c0 / CPR, p.m - 1)) * p.k + 8 * (c0 % CPR);
    const uint64_t aoff1 = static_cast<uint64_t>(min(m0 + c1 / CPR, p.m - 1)) * p.k + 8 * (c1 % CPR);
    const uint32_t bi = KS == 32 ? tid % 32 : tid % 64;
    const uint32_t bt = min(n0 / 16 + (KS == 32 ? tid / 32 : tid / 64), n_tiles - 1);
    const uint32_t bt2 = min(n0 / 16 + tid / 64 + 4, n_tiles - 1);  // 64-k stages
    const uint32_t scol_ld = min(n0 + tid % kTile, n - 1);  // the scale this thread stages
    // (slots travel by value: a slot passed by reference would be placed in
    // LDS by the compiler)
    auto load_stage = [&](uint32_t st) -> StageRegs {
        StageRegs r;
        const uint32_t k0 = kbeg + st * KS;
        r.h0 = *reinterpret_cast<const uint4*>(p.ahi + aoff0 + k0);
        r.l0 = *reinterpret_cast<const uint4*>(p.alo + aoff0 + k0);
        if constexpr (BM * CPR == 512) {
            r.h1 = *reinterpret_cast<const uint4*>(p.ahi + aoff1 + k0);
            r.l1 = *reinterpret_cast<const uint4*>(p.alo + aoff1 + k0);
        }
        r.sc = scales[static_cast<uint64_t>(scol_ld) * p.groups + k0 / p.group];
        const uint32_t sb = k0 / 128;
        if constexpr (KS == 32) {
            const uint32_t t = (k0 % 128) / kStepK, s = t / 2;
            const uint32_t L = (2 * (t % 2) + bi / 16) * 16 + bi % 16;
            const uint64_t tile = static_cast<uint64_t>(bt) * p.sb_total + sb;
            if constexpr (BITS == 4) {
                const uint2 w = *reinterpret_cast<const uint2*>(tiles + tile * 1024 + L * 16 + s * 8);
                r.b = make_uint4(w.x, w.y, 0u, 0u);
            } else {
                r.b = *reinterpret_cast<const uint4*>(tiles + tile * 2048 + s * 1024 + L * 16);
            }
        } else {
            const uint32_t s = (k0 % 128) / 64, L = bi;
            const uint64_t t0 = static_cast<uint64_t>(bt) * p.sb_total + sb;
            const uint64_t t1 = static_cast<uint64_t>(bt2) * p.sb_total + sb;
            if constexpr (BITS == 4) {
                const uint2 w0 = *reinterpret_cast<const uint2*>(tiles + t0 * 1024 + L * 16 + s * 8);
                const uint2 w1 = *reinterpret_cast<const uint2*>(tiles + t1 * 1024 + L * 16 + s * 8);
                r.b = make_uint4(w0.x, w0.y, w1.x, w1.y);
            } else {
                r.b = *reinterpret_cast<const uint4*>(tiles + t0 * 2048 + s * 1024 + L * 16);
                r.b2 = *reinterpret_cast<const uint4*>(tiles + t1 * 2048 + s * 1024 + L * 16);
            }
        }
        return r;
    };
    // 16 codes (INT4: words x, y; INT8: x, y, z, w) as fp16 at dst, each
    // group of 8 in the order kPerm8
    auto put_codes = [&](_Float16* dst, uint32_t x, uint32_t y, uint32_t z, uint32_t w) {
        *reinterpret_cast<v8h*>(dst) = BITS == 4 ? codes8<4>(x, 0u) : codes8<8>(x, y);
        *reinterpret_cast<v8h*>(dst + 8) = BITS == 4 ? codes8<4>(y, 0u) : codes8<8>(z, w);
    };
    auto store_stage = [&](int buf, StageRegs r) {
        const uint4 rb = r.b;
        if (tid < kTile) ss[buf][tid] = r.sc;
        *reinterpret_cast<uint4*>(&as[buf][0][c0 / CPR][8 * (c0 % CPR)]) = r.h0;
        *reinterpret_cast<uint4*>(&as[buf][1][c0 / CPR][8 * (c0 % CPR)]) = r.l0;
        if constexpr (BM * CPR == 512) {
            *reinterpret_cast<uint4*>(&as[buf][0][c1 / CPR][8 * (c1 % CPR)]) = r.h1;
            *reinterpret_cast<uint4*>(&as[buf][1][c1 / CPR][8 * (c1 % CPR)]) = r.l1;
        }
        if constexpr (KS == 32) {
            // 16 codes of column (tid / 32) * 16 + bi % 16, k 16 (bi / 16) .. + 15
            put_codes(&bs[buf][(tid / 32) * 16 + bi % 16][16 * (bi / 16)], rb.x, rb.y, rb.z, rb.w);
        } else if constexpr (BITS == 4) {
            // lane bi of tiles tid / 64 and tid / 64 + 4: column 16 t + bi % 16, k 16 (bi / 16) ..
            put_codes(&bs[buf][(tid / 64) * 16 + bi % 16][16 * (bi / 16)], rb.x, rb.y, 0u, 0u);
            put_codes(&bs[buf][(tid / 64 + 4) * 16 + bi % 16][16 * (bi / 16)], rb.z, rb.w, 0u, 0u);
        } else {
            const uint4 rb2 = r.b2;
            put_codes(&bs[buf][(tid / 64) * 16 + bi % 16][16 * (bi / 16)], rb.x, rb.y, rb.z, rb.w);
            put_codes(&bs[buf][(tid / 64 + 4) * 16 + bi % 16][16 * (bi / 16)], rb2.x, rb2.y, rb2.z, rb2.w);
        }
    };

    v4f acc[MT][4], tmp[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
            tmp[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
        }

    // Stages go global -> registers -> LDS through two register slots: the
    // loads of stage st + 2 are issued at step st and stored to LDS at the
    // end of step st + 1. Two slots keep the kernel within 256 registers, so
    // two blocks share each CU (their LDS, 73 KB each, fits twice) and one
    // block's MFMA work covers the other's loads, conversions and barriers:
    // [14336 x 4096] at M = 512 took 288 us with four slots and one block per
    // CU, 200 us so. steps is even (k % 128 == 0).
    StageRegs r0 = load_stage(0), r1 = load_stage(1);
    store_stage(0, r0);
    __syncthreads();
    // One stage. FRESH: the first stage of a group (its first product
    // starts the group's sums from zero); END: 1 the last stage of a group,
    // -1 decided at run time (GS == 0, where the group sums are cleared).
    auto step = [&](auto fresh_c, auto end_c, uint32_t st, StageRegs mine, StageRegs next) -> StageRegs {
        constexpr bool FRESH = decltype(fresh_c)::value;
        constexpr int END = decltype(end_c)::value;
        const int buf = st & 1;
        // this slot's stage is in LDS already; past the end the last stage
        // is loaded again, so every step issues the same loads and the
        // compiler's waits stay exact (a conditional load makes it wait for
        // every outstanding one where the paths join)
        mine = load_stage(min(st + 2, steps - 1));
        // operands of MFMA step h: A rows (BM / 2) wm + 16 i + lane % 16, B columns
        // 64 wn + 16 j + lane % 16, k 32 h + 8 (lane / 16) .. + 7 of the stage
#pragma unroll
        for (int h = 0; h < KS / kStepK; ++h) {
            const int kq = kStepK * h + 8 * (lane / 16);
            v8h bq[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bq[j] = *reinterpret_cast<const v8h*>(&bs[buf][64 * wn + 16 * j + lane % 16][kq]);
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const v8h ah = *reinterpret_cast<const v8h*>(&as[buf][0][(BM / 2) * wm + 16 * i + lane % 16][kq]);
                const v8h al = *reinterpret_cast<const v8h*>(&as[buf][1][(BM / 2) * wm + 16 * i + lane % 16][kq]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const v4f c = FRESH && h == 0 ? v4f{0.f, 0.f, 0.f, 0.f} : tmp[i][j];
                    tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq[j], c, 0, 0, 0);
                    tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq[j], tmp[i][j], 0, 0, 0);
                }
            }
        }
        if (END == 1 || (END == -1 && st % group_steps == group_steps - 1)) {
            // the group's scales, staged with this step's operands
            float sv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) sv[j] = ss[buf][64 * wn + 16 * j + lane % 16];
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(tmp[i][j][e], sv[j], acc[i][j][e]);
                    if constexpr (END == -1) tmp[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
                }
        }
        store_stage(buf ^ 1, next);  // after the last step: into a buffer nothing reads
        __syncthreads();
        return mine;
    };
    using T = std::true_type;
    using F = std::false_type;
    using E1 = std::integral_constant<int, 1>;
    using E0 = std::integral_constant<int, 0>;
    using ER = std::integral_constant<int, -1>;
    if constexpr (GS == 4) {
        for (uint32_t st = 0; st < steps; st += 4) {
            r0 = step(T{}, E0{}, st, r0, r1);
            r1 = step(F{}, E0{}, st + 1, r1, r0);
            r0 = step(F{}, E0{}, st + 2, r0, r1);
            r1 = step(F{}, E1{}, st + 3, r1, r0);
        }
    } else if constexpr (GS == 2) {
        for (uint32_t st = 0; st < steps; st += 2) {
            r0 = step(T{}, E0{}, st, r0, r1);
            r1 = step(F{}, E1{}, st + 1, r1, r0);
        }
    } else {
        for (uint32_t st = 0; st < steps; st += 2) {
            r0 = step(F{}, ER{}, st, r0, r1);
            r1 = step(F{}, ER{}, st + 1, r1, r0);
        }
    }

    // lane holds rows 4 (lane / 16) + e of each row tile, column lane % 16
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t row = m0 + (BM / 2) * wm + 16 * i + 4 * (lane / 16) + e;
            if (row >= p.m) continue;
            const int sh = p.row_exp[row] - kExpBias;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t col = n0 + 64 * wn + 16 * j + lane % 16;
                if (col >= n) continue;
                const uint64_t o = static_cast<uint64_t>(row) * n + col;
                const float val = ldexpf(acc[i][j][e], sh);
                if (gridDim.z > 1) {
                    p.partial[static_cast<uint64_t>(bz) * p.m * n + o] = val;
                    continue;
                }
                if (out != nullptr) out[o] = val;
                if (out2 != nullptr) out2[o] = resid[o] + val;
            }
        }
}

}  // namespace

namespace {

// hi and lo (fp16, m x k each), then the row exponents, in the workspace
struct SplitLayout {
    uint64_t lo_at, exp_at, floats;
};
SplitLayout split_layout(uint64_t m, uint64_t k) {
    const uint64_t half_floats = (m * k + 1) / 2;  // one array of m * k halves, in floats
    const uint64_t lo_at = (half_floats + 63) / 64 * 64, exp_at = lo_at + (half_floats + 63) / 64 * 64;
    return {lo_at, exp_at, exp_at + m};
}

}  // namespace

bool qgemm_mfma_takes(const float* a, const QuantWeight* const* w, uint32_t nseg, uint64_t m, const Workspace& ws) {
    if (nseg == 0 || nseg > kFusedMaxSegs || !aligned16(a) || m == 0 || m > 0xffffffffull) return false;
    const QuantWeight& w0 = *w[0];
    uint64_t blocks = 0;
    for (uint32_t i = 0; i < nseg; ++i) {
        const QuantWeight& x = *w[i];
        if (x.layout != QuantLayout::Mfma || x.k != w0.k || x.group != w0.group || x.format != w0.format ||
            x.k % 128 != 0 || x.group % kStepK != 0 || x.k % x.group != 0 || x.n > 0xffffffffull ||
            x.k > 0xffffffffull || x.tiles == nullptr)
            return false;
        blocks += (x.n + kTile - 1) / kTile;
    }
    return blocks <= 0xffffffffull && split_layout(m, w0.k).floats <= ws.floats;
}

bool qgemm_norm_takes(uint64_t k, const float* gamma) { return gamma != nullptr && aligned16(gamma) && k <= 2048 * 4; }

hipError_t launch_qgemm_multi(const float* a, const QuantWeight* const* w, float* const* out, uint32_t nseg,
                              uint64_t m, const Workspace& ws, hipStream_t s, const float* u,
                              const float* const* resid, float* const* out2, const float* gamma, float eps) {
    if (!qgemm_mfma_takes(a, w, nseg, m, ws)) return hipErrorNotSupported;
    const QuantWeight& w0 = *w[0];
    if (gamma != nullptr && (u != nullptr || !qgemm_norm_takes(w0.k, gamma))) return hipErrorNotSupported;
    const SplitLayout lay = split_layout(m, w0.k);
    _Float16* hi = reinterpret_cast<_Float16*>(ws.data);
    _Float16* lo = reinterpret_cast<_Float16*>(ws.data + lay.lo_at);
    int* row_exp = reinterpret_cast<int*>(ws.data + lay.exp_at);
    // rows of up to 32768 elements stay in registers between the passes
    const uint32_t kk = static_cast<uint32_t>(w0.k);
    const dim3 sgrid(static_cast<unsigned>(m));
    if (w0.k <= 2048 * 4) split_rows<4><<<sgrid, 256, 0, s>>>(a, u, hi, lo, row_exp, kk, gamma, eps);
    else if (w0.k <= 2048 * 8) split_rows<8><<<sgrid, 256, 0, s>>>(a, u, hi, lo, row_exp, kk, nullptr, 0.f);
    else if (w0.k <= 2048 * 16) split_rows<16><<<sgrid, 256, 0, s>>>(a, u, hi, lo, row_exp, kk, nullptr, 0.f);
    else split_rows<0><<<sgrid, 256, 0, s>>>(a, u, hi, lo, row_exp, kk, nullptr, 0.f);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    GemmArgs p{};
    p.ahi = hi;
    p.alo = lo;
    p.row_exp = row_exp;
    uint32_t blocks = 0;
    for (uint32_t i = 0; i < nseg; ++i) {
        const bool res = resid != nullptr && out2 != nullptr && out2[i] != nullptr;
        p.seg[i] = GemmSeg{w[i]->tiles, w[i]->scales, out[i], res ? resid[i] : nullptr, res ? out2[i] : nullptr,
                           static_cast<uint32_t>(w[i]->n), blocks};
        blocks += static_cast<uint32_t>((w[i]->n + kTile - 1) / kTile);
    }
    p.nseg = nseg;
    p.m = static_cast<uint32_t>(m);
    p.k = static_cast<uint32_t>(w0.k);
    p.group = w0.group;
    p.groups = static_cast<uint32_t>(w0.k / w0.group);
    p.sb_total = static_cast<uint32_t>(w0.k / 128);
    // 128-row blocks, or 64-row ones (three per CU, each with less operand
    // reuse) when 128-row blocks would not give every CU one. Measured on
    // MI355X: M = 1024 [4096 x 4096] (256 blocks of 128 rows) runs faster in
    // 64-row blocks; M = 512 [14336 x 4096] (448) runs slower (200 -> 250 us).
    // 128-row blocks, or when they would not give every CU one: k in two
    // slices of 128-row blocks (one weight, the slice a whole number of
    // groups and 128-k superblocks, room for the partial sums), else 64-row
    // blocks. Measured on MI355X at M = 1024: [4096 x 14336] 395-402 us in
    // k slices (the slice sums included) against 440 us in 64-row blocks.
    const uint64_t blocks128 = static_cast<uint64_t>(blocks) * ((m + 127) / 128);
    const uint64_t part_at = (lay.floats + 63) / 64 * 64;
    const bool sliced = blocks128 <= compute_units() && nseg == 1 && (w0.k / 2) % 128 == 0 &&
                        (w0.k / 2) % w0.group == 0 && part_at + 2 * m * w0.n <= ws.floats;
    const bool rows64 = blocks128 <= compute_units() && !sliced;
    const bool deep = rows64 && w0.group % 64 == 0;  // 64-k stages
    p.partial = sliced ? ws.data + part_at : nullptr;
    const dim3 grid(blocks, static_cast<unsigned>(rows64 ? (m + 63) / 64 : (m + 127) / 128), sliced ? 2u : 1u);
    // stages per group when it is a compile-time form: 128 / KS for group 128
    // (4 or 2), 2 for group 64 in 32-k stages; 0 otherwise
    const int ks = deep ? 64 : 32;
    const int gs = w0.group == 128 ? 128 / ks : w0.group == 64 && ks == 32 ? 2 : 0;
#define SL_QGEMM(B, R, K)                                                    \
    do {                                                                     \
        if (gs == 4) qgemm_mfma<B, R, K, 4><<<grid, 256, 0, s>>>(p);          \
        else if (gs == 2) qgemm_mfma<B, R, K, 2><<<grid, 256, 0, s>>>(p);     \
        else qgemm_mfma<B, R, K, 0><<<grid, 256, 0, s>>>(p);                  \
    } while (0)
    if (w0.format == SL_QFORMAT_INT4) {
        if (deep) SL_QGEMM(4, 64, 64);
        else if (rows64) SL_QGEMM(4, 64, 32);
        else SL_QGEMM(4, 128, 32);
    } else {
        if (deep) SL_QGEMM(8, 64, 64);
        else if (rows64) SL_QGEMM(8, 64, 32);
        else SL_QGEMM(8, 128, 32);
    }
#undef SL_QGEMM
    if (sliced) {
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        const bool res = resid != nullptr && out2 != nullptr && out2[0] != nullptr;
        const uint64_t count = m * w0.n;
        gemm_slices_sum<<<grid_for(count, 256, 4096), 256, 0, s>>>(p.partial, 2, count, out[0],
                                                                  res ? resid[0] : nullptr, res ? out2[0] : nullptr);
    }
    return hipGetLastError();
}

hipError_t launch_qgemm_mfma(const float* a, const QuantWeight& w, float* out, uint64_t m, const Workspace& ws,
                             hipStream_t s) {
    const QuantWeight* ws1[1] = {&w};
    float* outs[1] = {out};
    return launch_qgemm_multi(a, ws1, outs, 1, m, ws, s);
}

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_qgemm_mfma() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_rows<0>));
}

}  // namespace slhip
