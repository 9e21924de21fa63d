// Dense f32 MatMulNT / MatMulNN (reference/matmul.rs:29-110) with the
// equal-or-one batch broadcast of device.rs:1357-1407.
//
// sgemm_mfma (k a multiple of 4, 16-byte aligned operands, and for NN n a
// multiple of 4): f32 matrix cores, v_mfma_f32_16x16x4_f32. A 256-thread
// block computes a 128x128 output tile, each wave a 64x64 quadrant as 4x4
// accumulator tiles of 16x16. K is staged 16 at a time through two LDS
// buffers ([row][k], 16 k + 4 pad floats per row), the next stage's
// float4s waiting in registers. Lane l of an MFMA supplies A[l % 16][k] and
// B[k][l % 16]; lane group g = l / 16 takes k = 4 g + s at step s of a stage,
// so one 16-byte LDS read per operand tile feeds four MFMAs. Products and
// sums are f32 (the hardware's sum order, not ascending k), within the 1e-4
// normwise bound.
//
// sgemm_tiled (every other shape): a 64x64 tile per 256-thread block, a 4x4
// register micro-tile per thread, K by 16 through LDS; any shape, both B
// layouts, any alignment. Products accumulate with fmaf in ascending k.
#include "common.h"
#include "kernels.h"

namespace slhip {
namespace {

constexpr int BM = 64, BN = 64, BK = 16;

typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kTile = 128, kStage = 16, kRow = kStage + 4;  // LDS row: 16 k + 4 pad floats

template <bool NT>
__global__ __launch_bounds__(256) void sgemm_mfma(const float* __restrict__ a, const float* __restrict__ b,
                                                  float* __restrict__ out, uint32_t m, uint32_t k, uint32_t n,
                                                  uint64_t a_batch_stride, uint64_t b_batch_stride,
                                                  uint64_t batch_base) {
    __shared__ __align__(16) float as[2][kTile][kRow];
    __shared__ __align__(16) float bs[2][kTile][kRow];
    const uint64_t z = batch_base + blockIdx.z;
    a += z * a_batch_stride;
    b += z * b_batch_stride;
    out += z * m * static_cast<uint64_t>(n);
    const uint32_t row0 = blockIdx.y * kTile, col0 = blockIdx.x * kTile;
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wr = wave / 2, wc = wave % 2;  // the wave's 64x64 quadrant

    // One stage: A rows [row0, row0 + 128) x k [k0, k0 + 16) as 512 float4,
    // two per thread (row tid / 4 + 64 i, k 4 (tid % 4)); B the same for NT
    // ([n][k] rows), and for NN 16 k rows of 128 columns (k tid / 32 + 8 i,
    // columns 4 (tid % 32)). Past m, n or k: zeros.
    v4f ra[2], rb[2];
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t r = static_cast<uint32_t>(tid / 4 + 64 * i), gk = k0 + 4 * (tid % 4);
            ra[i] = row0 + r < m && gk < k ? *reinterpret_cast<const v4f*>(a + static_cast<uint64_t>(row0 + r) * k + gk)
                                           : zero;
            if constexpr (NT) {
                rb[i] = col0 + r < n && gk < k
                            ? *reinterpret_cast<const v4f*>(b + static_cast<uint64_t>(col0 + r) * k + gk)
                            : zero;
            } else {
                const uint32_t kk = k0 + static_cast<uint32_t>(tid / 32 + 8 * i), gn = col0 + 4 * (tid % 32);
                rb[i] = kk < k && gn < n ? *reinterpret_cast<const v4f*>(b + static_cast<uint64_t>(kk) * n + gn) : zero;
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = tid / 4 + 64 * i;
            *reinterpret_cast<v4f*>(&as[buf][r][4 * (tid % 4)]) = ra[i];
            if constexpr (NT) {
                *reinterpret_cast<v4f*>(&bs[buf][r][4 * (tid % 4)]) = rb[i];
            } else {
                const int kk = tid / 32 + 8 * i, c = 4 * (tid % 32);
#pragma unroll
                for (int j = 0; j < 4; ++j) bs[buf][c + j][kk] = rb[i][j];
            }
        }
    };

    v4f acc[4][4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[s][t] = zero;
    const int lr = lane % 16, lk = 4 * (lane / 16);
    load(0);
    store(0);
    __syncthreads();
    int buf = 0;
    for (uint32_t k0 = 0; k0 < k; k0 += kStage) {
        const bool more = k0 + kStage < k;
        if (more) load(k0 + kStage);
        v4f va[4], vb[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) va[s] = *reinterpret_cast<const v4f*>(&as[buf][wr * 64 + s * 16 + lr][lk]);
#pragma unroll
        for (int t = 0; t < 4; ++t) vb[t] = *reinterpret_cast<const v4f*>(&bs[buf][wc * 64 + t * 16 + lr][lk]);
#pragma unroll
        for (int step = 0; step < 4; ++step)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    acc[s][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[s][step], vb[t][step], acc[s][t], 0, 0, 0);
        if (more) {
            store(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }
    }
    // accumulator value i of lane l: row 4 (l / 16) + i, column l % 16 of its 16x16 tile
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t gr = row0 + wr * 64 + s * 16 + 4 * (lane / 16) + i;
            if (gr >= m) continue;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t gc = col0 + wc * 64 + t * 16 + lr;
                if (gc < n) out[static_cast<uint64_t>(gr) * n + gc] = acc[s][t][i];
            }
        }
}

template <bool NT>
__global__ __launch_bounds__(256) void sgemm_tiled(const float* __restrict__ a, const float* __restrict__ b,
                                                   float* __restrict__ out, uint64_t m, uint64_t k, uint64_t n,
                                                   uint64_t a_batch_stride, uint64_t b_batch_stride,
                                                   uint64_t batch_base) {
    __shared__ float as[BK][BM + 4];
    __shared__ float bs[BK][BN + 4];
    const uint64_t z = batch_base + blockIdx.z;
    a += z * a_batch_stride;
    b += z * b_batch_stride;
    out += z * m * n;
    const uint64_t row0 = static_cast<uint64_t>(blockIdx.y) * BM;
    const uint64_t col0 = static_cast<uint64_t>(blockIdx.x) * BN;
    const int tid = threadIdx.x;
    const int ty = tid / 16, tx = tid % 16;
    float acc[4][4] = {};

    for (uint64_t k0 = 0; k0 < k; k0 += BK) {
        // A tile: 64 rows x 16 k -> as[k][row]
        for (int e = tid; e < BM * BK; e += 256) {
            const int r = e / BK, c = e % BK;
            const uint64_t gr = row0 + r, gc = k0 + c;
            as[c][r] = (gr < m && gc < k) ? a[gr * k + gc] : 0.f;
        }
        // B tile: bs[k][col]
        for (int e = tid; e < BN * BK; e += 256) {
            if (NT) {
                const int r = e / BK, c = e % BK;  // r: col of out, c: k
                const uint64_t gn = col0 + r, gk = k0 + c;
                bs[c][r] = (gn < n && gk < k) ? b[gn * k + gk] : 0.f;
            } else {
                const int c = e / BN, r = e % BN;  // c: k, r: col
                const uint64_t gn = col0 + r, gk = k0 + c;
                bs[c][r] = (gn < n && gk < k) ? b[gk * n + gn] : 0.f;
            }
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

}  // namespace

hipError_t launch_matmul(const float* a, const float* b, float* out, uint64_t batch, uint64_t batch_a,
                         uint64_t batch_b, uint64_t m, uint64_t k, uint64_t n, bool nt, hipStream_t s) {
    if (batch == 0 || m == 0 || n == 0) return hipSuccess;
    const uint64_t a_stride = batch_a == 1 && batch > 1 ? 0 : m * k;
    const uint64_t b_stride = batch_b == 1 && batch > 1 ? 0 : n * k;
    // matrix cores: 16-byte rows (k % 4 == 0, and n % 4 == 0 for NN rows of
    // B), 16-byte aligned operands, 32-bit extents, a grid y within 65535
    // row tiles, and at least 32 rows (fewer would leave most of a 128-row
    // tile's products unused)
    const bool mfma = k % 4 == 0 && k > 0 && (nt || n % 4 == 0) && aligned16(a) && aligned16(b) && m >= 32 &&
                      m <= 65535ull * kTile && n <= 0xffffffffull && k <= 0xffffffffull;
    if (mfma) {
        const unsigned gx = static_cast<unsigned>((n + kTile - 1) / kTile);
        const unsigned gy = static_cast<unsigned>((m + kTile - 1) / kTile);
        for (uint64_t base = 0; base < batch; base += 65535) {
            const unsigned gz = static_cast<unsigned>(batch - base < 65535 ? batch - base : 65535);
            const dim3 grid(gx, gy, gz);
            const uint32_t m32 = static_cast<uint32_t>(m), k32 = static_cast<uint32_t>(k), n32 = static_cast<uint32_t>(n);
            if (nt) sgemm_mfma<true><<<grid, 256, 0, s>>>(a, b, out, m32, k32, n32, a_stride, b_stride, base);
            else sgemm_mfma<false><<<grid, 256, 0, s>>>(a, b, out, m32, k32, n32, a_stride, b_stride, base);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const unsigned gx = static_cast<unsigned>((n + BN - 1) / BN);
    const unsigned gy = static_cast<unsigned>((m + BM - 1) / BM);
    for (uint64_t base = 0; base < batch; base += 65535) {
        const unsigned gz = static_cast<unsigned>(batch - base < 65535 ? batch - base : 65535);
        dim3 grid(gx, gy, gz);
        if (nt) sgemm_tiled<true><<<grid, 256, 0, s>>>(a, b, out, m, k, n, a_stride, b_stride, base);
        else sgemm_tiled<false><<<grid, 256, 0, s>>>(a, b, out, m, k, n, a_stride, b_stride, base);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_matmul() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&sgemm_tiled<true>));
}

}  // namespace slhip
