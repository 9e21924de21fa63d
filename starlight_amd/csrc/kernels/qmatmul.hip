// Group-quantized MatMulNT: out[m, n] = sum_k a[m, k] * (q[n, k] * s[n, k / G]).
//
// No reference kernel exists for this (sl-precision is absent from the
// reference); the result must equal matmul_nt(a, dequant(q, s))
// (reference/matmul.rs:29-59) within the normwise 1e-4 bound, and the decode
// of each code is exact.
//
// Device-private layouts (made by launch_quant_repack from the uploaded
// payload):
//  * Mfma (k % 128 == 0, group % 64 == 0): 16-row x 128-k superblocks in the
//    MFMA operand order described in qgemv_mfma.hip — every shape the
//    llama configurations use;
//  * RowMajor (anything else): the payload bytes with every code stored
//    offset-binary, u = q + 8 (INT4 nibble) or u = q + 128 (INT8 byte), i.e.
//    the payload XOR 0x88 / 0x80. Offset-binary codes convert to f32 with one
//    v_cvt_f32_ubyte per element after a mask, and the offset is removed once
//    per 32-element chunk: sum_k q*x = sum_k u*x - off * sum_k x.
//
// Kernels
//  * qgemv_mfma (qgemv_mfma.hip) — m <= 16 on the Mfma layout;
//  * qgemv_valu — m <= 16 on the RowMajor layout: one wave owns 4 weight
//    rows; lanes walk 16-byte chunks of those rows, so a wave's load covers
//    1 KiB of one row contiguously; x chunks are shared by the 4 rows;
//  * qgemm_mfma (qgemm_mfma.hip) — m > 16 on the Mfma layout: fp16 matrix
//    cores on split activations;
//  * qgemm_tiled — large m otherwise: the SGEMM tile loop with the B tile
//    decoded into LDS as f32 (either layout);
//  * qmm_generic — any geometry (correctness path, either layout).
#include "common.h"
#include "kernels.h"
#include "starlight_hip.h"

namespace slhip {
namespace {

__global__ void xor_words(const uint32_t* __restrict__ in, uint32_t* __restrict__ out, uint64_t words,
                          uint32_t mask) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride)
        out[i] = in[i] ^ mask;
}

__device__ __forceinline__ float ubyte(uint32_t w, int i) {
    return static_cast<float>((w >> (8 * i)) & 0xffu);
}

// Sum of u*x over the 32 INT4 codes of one 16-byte chunk (8 per word;
// byte j of a word holds k = 2j in its low and k = 2j + 1 in its high nibble).
__device__ __forceinline__ float dot_chunk_int4(uint4 w, const float* x) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = words[i] & 0x0F0F0F0Fu;
        const uint32_t hi = (words[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            d = fmaf(ubyte(lo, j), x[8 * i + 2 * j], d);
            d = fmaf(ubyte(hi, j), x[8 * i + 2 * j + 1], d);
        }
    }
    return d;
}

// Sum of u*x over the 16 INT8 codes of one 16-byte chunk.
__device__ __forceinline__ float dot_chunk_int8(uint4 w, const float* x) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) d = fmaf(ubyte(words[i], j), x[4 * i + j], d);
    return d;
}

constexpr int kRowsPerWave = 4;

// grid: (ceil(n / (4 waves * 4 rows)), m). Requires k % group == 0,
// group % CK == 0 and 16-byte aligned rows (k % CK == 0).
template <int BITS>
__global__ __launch_bounds__(256) void qgemv_valu(const float* __restrict__ a, const uint8_t* __restrict__ tiles,
                                                  const float* __restrict__ scales, float* __restrict__ out,
                                                  uint32_t n, uint32_t k, uint32_t group) {
    prefetch_kernarg<arg_bytes<const float*, const uint8_t*, const float*, float*, uint32_t, uint32_t, uint32_t>()>();
    constexpr int CK = BITS == 4 ? 32 : 16;        // codes per 16-byte chunk
    constexpr float OFF = BITS == 4 ? 8.f : 128.f;  // offset-binary bias
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t row0 = (blockIdx.x * 4 + threadIdx.x / kWave) * kRowsPerWave;
    if (row0 >= n) return;
    const uint64_t mrow = blockIdx.y;
    const float* x = a + mrow * k;
    const uint32_t chunks = k / CK;
    const uint32_t row_bytes = BITS == 4 ? k / 2 : k;
    const uint32_t groups = k / group;
    float acc[kRowsPerWave] = {};
    for (uint32_t c = lane; c < chunks; c += kWave) {
        float xv[CK];
        const float4* x4 = reinterpret_cast<const float4*>(x + static_cast<uint64_t>(c) * CK);
#pragma unroll
        for (int i = 0; i < CK / 4; ++i) {
            const float4 v = x4[i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
        float xs = 0.f;
#pragma unroll
        for (int i = 0; i < CK; ++i) xs += xv[i];
        const uint32_t g = c * CK / group;
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
            const uint32_t row = row0 + r;
            if (row >= n) break;
            const uint4 w = *reinterpret_cast<const uint4*>(tiles + static_cast<uint64_t>(row) * row_bytes +
                                                            static_cast<uint64_t>(c) * 16);
            const float d = BITS == 4 ? dot_chunk_int4(w, xv) : dot_chunk_int8(w, xv);
            const float part = fmaf(-OFF, xs, d);
            acc[r] = fmaf(part, scales[static_cast<uint64_t>(row) * groups + g], acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < n) out[mrow * n + row0 + r] = v;
    }
}

// Integer code of weight (r, c) in either private layout.
__device__ __forceinline__ float decode(const uint8_t* tiles, uint32_t bits, uint64_t row_bytes, uint64_t r,
                                        uint64_t c, bool mfma, uint64_t sb_total) {
    if (mfma) {
        const uint64_t nt = r / 16, sb = c / 128;
        const uint32_t s = (c % 128) / 64, lane = static_cast<uint32_t>(((c % 64) / 16) * 16 + r % 16);
        const uint32_t j = c % 16;
        if (bits == 4) {
            const uint8_t byte = tiles[(nt * sb_total + sb) * 1024 + lane * 16 + s * 8 + (j < 8 ? 0 : 4) + (j & 3)];
            const int u = (j & 4) ? byte >> 4 : byte & 0x0F;  // two's complement nibble
            return static_cast<float>(u >= 8 ? u - 16 : u);
        }
        return static_cast<float>(
            static_cast<int8_t>(tiles[(nt * sb_total + sb) * 2048 + s * 1024 + lane * 16 + j]));
    }
    if (bits == 4) {
        const uint8_t byte = tiles[r * row_bytes + c / 2];
        const int u = (c & 1) ? byte >> 4 : byte & 0x0F;
        return static_cast<float>(u - 8);
    }
    return static_cast<float>(static_cast<int>(tiles[r * row_bytes + c]) - 128);
}

// Payload code (two's complement, row-major) of weight (r, c).
__device__ __forceinline__ int payload_code(const uint8_t* payload, uint32_t bits, uint64_t k, uint64_t r,
                                            uint64_t c) {
    if (bits == 4) {
        const uint8_t byte = payload[r * ((k + 1) / 2) + c / 2];
        const int nib = (c & 1) ? byte >> 4 : byte & 0x0F;
        return nib >= 8 ? nib - 16 : nib;
    }
    return static_cast<int8_t>(payload[r * k + c]);
}

// One thread per 32-bit word of the Mfma layout (see qgemv_mfma.hip).
__global__ void repack_mfma(const uint8_t* __restrict__ payload, uint32_t* __restrict__ tiles, uint32_t bits,
                            uint64_t n, uint64_t k, uint64_t words) {
    const uint64_t sb_total = k / 128;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t w = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < words; w += stride) {
        uint32_t out = 0;
        if (bits == 4) {
            const uint64_t tile = w / 256, within = w % 256;
            const uint64_t nt = tile / sb_total, sb = tile % sb_total;
            const uint32_t lane = static_cast<uint32_t>(within / 4), wi = static_cast<uint32_t>(within % 4);
            const uint32_t s = wi / 2, half = wi % 2;
            const uint64_t r = nt * 16 + lane % 16;
            for (uint32_t jj = 0; jj < 8; ++jj) {
                const uint32_t j = half * 8 + jj;
                const uint64_t c = sb * 128 + s * 64 + (lane / 16) * 16 + j;
                // two's complement nibble; rows past n are zero
                const uint32_t u = r < n ? static_cast<uint32_t>(payload_code(payload, 4, k, r, c)) & 0xFu : 0u;
                const uint32_t nib = jj < 4 ? 2 * jj : 2 * (jj - 4) + 1;
                out |= (u & 0xF) << (4 * nib);
            }
        } else {
            const uint64_t tile = w / 512, within = w % 512;
            const uint64_t nt = tile / sb_total, sb = tile % sb_total;
            const uint32_t s = static_cast<uint32_t>(within / 256);
            const uint32_t lane = static_cast<uint32_t>((within % 256) / 4), wq = static_cast<uint32_t>(within % 4);
            const uint64_t r = nt * 16 + lane % 16;
            for (uint32_t b = 0; b < 4; ++b) {
                const uint64_t c = sb * 128 + s * 64 + (lane / 16) * 16 + 4 * wq + b;
                const uint32_t q = r < n ? static_cast<uint32_t>(payload_code(payload, 8, k, r, c)) & 0xFFu : 0u;
                out |= q << (8 * b);
            }
        }
        tiles[w] = out;
    }
}

// One thread per output, any geometry.
__global__ __launch_bounds__(256) void qmm_generic(const float* __restrict__ a, const uint8_t* __restrict__ tiles,
                                                   const float* __restrict__ scales, float* __restrict__ out,
                                                   uint64_t m, uint64_t n, uint64_t k, uint32_t group,
                                                   uint32_t bits, bool mfma) {
    const uint64_t total = m * n;
    const uint64_t sb_total = k / 128;
    const uint64_t row_bytes = bits == 4 ? (k + 1) / 2 : k;
    const uint64_t groups = k / group;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        const uint64_t r = i / n, c = i % n;
        float acc = 0.f;
        for (uint64_t kk = 0; kk < k; ++kk)
            acc = fmaf(a[r * k + kk], decode(tiles, bits, row_bytes, c, kk, mfma, sb_total) *
                                          scales[c * groups + kk / group], acc);
        out[i] = acc;
    }
}

constexpr int BM = 64, BN = 64, BK = 16;

// Large-m path: SGEMM tiles with B decoded into LDS (w = q * s in f32).
__global__ __launch_bounds__(256) void qgemm_tiled(const float* __restrict__ a, const uint8_t* __restrict__ tiles,
                                                   const float* __restrict__ scales, float* __restrict__ out,
                                                   uint64_t m, uint64_t k, uint64_t n, uint32_t group,
                                                   uint32_t bits, bool mfma) {
    __shared__ float as[BK][BM + 4];
    const uint64_t sb_total = k / 128;
    __shared__ float bs[BK][BN + 4];
    const uint64_t row0 = static_cast<uint64_t>(blockIdx.y) * BM;
    const uint64_t col0 = static_cast<uint64_t>(blockIdx.x) * BN;
    const uint64_t row_bytes = bits == 4 ? (k + 1) / 2 : k;
    const uint64_t groups = k / group;
    const int tid = threadIdx.x;
    const int ty = tid / 16, tx = tid % 16;
    float acc[4][4] = {};
    for (uint64_t k0 = 0; k0 < k; k0 += BK) {
        for (int e = tid; e < BM * BK; e += 256) {
            const int r = e / BK, c = e % BK;
            const uint64_t gr = row0 + r, gc = k0 + c;
            as[c][r] = (gr < m && gc < k) ? a[gr * k + gc] : 0.f;
        }
        for (int e = tid; e < BN * BK; e += 256) {
            const int r = e / BK, c = e % BK;
            const uint64_t gn = col0 + r, gk = k0 + c;
            bs[c][r] = (gn < n && gk < k) ? decode(tiles, bits, row_bytes, gn, gk, mfma, sb_total) *
                                                scales[gn * groups + gk / group]
                                          : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                av[i] = as[kk][ty * 4 + i];
                bv[i] = bs[kk][tx * 4 + i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint64_t gr = row0 + ty * 4 + i;
        if (gr >= m) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint64_t gc = col0 + tx * 4 + j;
            if (gc < n) out[gr * n + gc] = acc[i][j];
        }
    }
}

// Scales per 128-k superblock of each 16-row tile, in the order a wave reads
// them: tile_scales[((tile * sb_total + sb) * 16 + r) * gps + j] is the scale
// of row 16 * tile + r for the j-th group of superblock sb (gps = 2 groups
// per superblock for group 64, else 1 and the group containing sb).
__global__ void scale_repack(const float* __restrict__ scales, float* __restrict__ tile_scales, uint64_t n,
                             uint64_t groups, uint64_t sb_total, uint32_t group, uint32_t gps, uint64_t total) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        const uint64_t j = i % gps, r = (i / gps) % 16, sb = (i / (16 * gps)) % sb_total;
        const uint64_t tile = i / (16 * gps * sb_total);
        const uint64_t row = tile * 16 + r;
        const uint64_t g = group <= 128 ? sb * gps + j : sb * 128 / group;
        tile_scales[i] = row < n ? scales[row * groups + g] : 0.f;
    }
}

}  // namespace

QuantLayout quant_layout_for(uint32_t format, uint64_t n, uint64_t k, uint32_t group) {
    (void)format;
    (void)n;
    if (group != 0 && k % 128 == 0 && group % 64 == 0 && k % group == 0 && group <= 4096) return QuantLayout::Mfma;
    return QuantLayout::RowMajor;
}

uint64_t quant_tile_bytes(uint32_t format, uint64_t n, uint64_t k, QuantLayout layout) {
    if (layout == QuantLayout::Mfma)
        return (n + 15) / 16 * (k / 128) * (format == SL_QFORMAT_INT4 ? 1024 : 2048);
    const uint64_t bytes = format == SL_QFORMAT_INT4 ? n * ((k + 1) / 2) : n * k;
    return (bytes + 3) / 4 * 4;
}

hipError_t launch_quant_repack(const uint8_t* payload, uint8_t* tiles, uint32_t format, uint64_t n, uint64_t k,
                               QuantLayout layout, hipStream_t s) {
    const uint64_t words = quant_tile_bytes(format, n, k, layout) / 4;
    if (words == 0) return hipSuccess;
    if (layout == QuantLayout::Mfma) {
        repack_mfma<<<grid_for(words, 256, 256 * 16), 256, 0, s>>>(payload, reinterpret_cast<uint32_t*>(tiles),
                                                                    format == SL_QFORMAT_INT4 ? 4 : 8, n, k, words);
        return hipGetLastError();
    }
    xor_words<<<grid_for(words, 256, 256 * 8), 256, 0, s>>>(
        reinterpret_cast<const uint32_t*>(payload), reinterpret_cast<uint32_t*>(tiles), words,
        format == SL_QFORMAT_INT4 ? 0x88888888u : 0x80808080u);
    return hipGetLastError();
}

uint64_t quant_tile_scale_floats(uint64_t n, uint64_t k, uint32_t group, QuantLayout layout) {
    if (layout != QuantLayout::Mfma || group == 0) return 0;
    const uint64_t gps = group < 128 ? 128 / group : 1;
    return (n + 15) / 16 * (k / 128) * 16 * gps;
}

hipError_t launch_scale_repack(const float* scales, float* tile_scales, uint64_t n, uint64_t k, uint32_t group,
                               hipStream_t s) {
    const uint64_t total = quant_tile_scale_floats(n, k, group, QuantLayout::Mfma);
    if (total == 0) return hipSuccess;
    const uint32_t gps = group < 128 ? 128 / group : 1;
    scale_repack<<<grid_for(total, 256, 256 * 64), 256, 0, s>>>(scales, tile_scales, n, k / group, k / 128, group,
                                                                gps, total);
    return hipGetLastError();
}

hipError_t launch_qmatmul(const float* a, const QuantWeight& w, float* out, uint64_t m, const Workspace& ws,
                          hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (w.k == 0) return launch_fill_zero(out, m * w.n, s);
    const uint32_t bits = w.format == SL_QFORMAT_INT4 ? 4 : 8;
    const bool mfma = w.layout == QuantLayout::Mfma;
    if (mfma && m <= 16 && aligned16(a)) {
        QgemvFused f{};
        f.a = a;
        f.w[0] = &w;
        f.out[0] = out;
        f.nseg = 1;
        f.m = m;
        f.epilogue = kFusedPlain;
        f.partial = ws.data;
        f.partial_floats = ws.floats;
        hipError_t e = launch_qgemv_fused(f, s);
        if (e != hipErrorNotSupported) return e;
        e = launch_qgemv_mfma(a, w, out, m, ws, s);
        if (e != hipErrorNotSupported) return e;
        (void)hipGetLastError();
    }
    if (mfma && m > 16) {
        const hipError_t e = launch_qgemm_mfma(a, w, out, m, ws, s);
        if (e != hipErrorNotSupported) return e;
    }
    const uint32_t ck = bits == 4 ? 32 : 16;
    const bool fast = !mfma && w.k % ck == 0 && w.group % ck == 0 && w.k % w.group == 0 && aligned16(a) &&
                      aligned16(w.tiles) && w.n <= 0xffffffffu && w.k <= 0xffffffffu;
    if (fast && m <= 16) {
        dim3 grid(static_cast<unsigned>((w.n + 4 * kRowsPerWave - 1) / (4 * kRowsPerWave)),
                  static_cast<unsigned>(m));
        if (bits == 4)
            qgemv_valu<4><<<grid, 256, 0, s>>>(a, w.tiles, w.scales, out, static_cast<uint32_t>(w.n),
                                               static_cast<uint32_t>(w.k), w.group);
        else
            qgemv_valu<8><<<grid, 256, 0, s>>>(a, w.tiles, w.scales, out, static_cast<uint32_t>(w.n),
                                               static_cast<uint32_t>(w.k), w.group);
        return hipGetLastError();
    }
    if (w.k % w.group == 0 && m > 16) {
        dim3 grid(static_cast<unsigned>((w.n + BN - 1) / BN), static_cast<unsigned>((m + BM - 1) / BM));
        qgemm_tiled<<<grid, 256, 0, s>>>(a, w.tiles, w.scales, out, m, w.k, w.n, w.group, bits, mfma);
        return hipGetLastError();
    }
    qmm_generic<<<grid_for(m * w.n, 256, 256 * 16), 256, 0, s>>>(a, w.tiles, w.scales, out, m, w.n, w.k,
                                                                 w.group, bits, mfma);
    return hipGetLastError();
}

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_qmatmul() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&xor_words));
}

}  // namespace slhip
