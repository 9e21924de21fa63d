// Group-quantized GEMV / skinny GEMM (m <= 16 activation rows) on the int8
// matrix cores: v_mfma_i32_16x16x64_i8.
//
// The f32 activations are turned into exact integers first: per block and
// row, x = X * 2^(E-22) with X = rint(x * 2^(22-E)), E the binary exponent of
// the row slice's max |x| (so |X| <= 2^22, element error <= 2^-23 max|x|),
// and X is split into three signed 8-bit limbs X = L0 + 2^8 L1 + 2^16 L2.
// The weight codes are small integers, so every limb product sum
// sum_k code * L_i is computed exactly in i32 by the MFMA; per group of G
// codes the three sums are combined in f32 and scaled by the group scale:
//   out[m, n] = 2^(E-22) * sum_g s[n, g] * sum_i 2^(8i) sum_{k in g} q[n, k] L_i[m, k].
// Only the final combination rounds, so the result matches
// matmul_nt(a, dequant(q, s)) (reference/matmul.rs:29-59) to about 1e-7
// normwise, well inside the 1e-4 bound.
//
// Weight tiles (QuantLayout::Mfma, built by launch_quant_repack): for each
// 16-row tile nt and 128-k superblock sb, one contiguous block in which lane l
// of a wave finds exactly its MFMA B operand for both 64-k steps:
//   INT4: 1024 bytes, lane l owns bytes [16l, 16l + 16): 8 bytes per step;
//         codes stored offset-binary (u = q + 8) and arranged so that
//         w & 0x0F0F0F0F and (w >> 4) & 0x0F0F0F0F give the operand bytes in
//         k order; the +8 offset is removed exactly with a per-group
//         integer correction 8 * sum_k X.
//   INT8: 2048 bytes, step s at 1024 s, lane l owns bytes [16l, 16l + 16).
// Operand k order within a step: lane l holds k = 16 (l / 16) + j, j < 16,
// for row l % 16 — identical for A and B, which is all the product needs.
//
// Work split: a block of 4 waves owns 4 adjacent 16-row tiles (one per wave)
// and one split of the K superblocks; when K is split across blocks, each
// block writes its partial tile to the workspace and the last block of a
// tile column (counted with one device-scope atomic per column) adds the
// partials in split order — deterministic, no extra launch, and the counter
// is returned to zero.
#include "common.h"
#include "kernels.h"
#include "starlight_hip.h"

namespace slhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWavesPerBlock = 4;
constexpr int kLdsLimbBytes = 48 * 1024;  // 3 limbs x m x k-slice

struct QgemvArgs {
    const float* a;
    const uint8_t* tiles;
    const float* scales;
    float* out;
    float* partial;      // [splits, m, n] when splits > 1
    uint32_t* counters;  // one per n-block
    uint32_t m, n, k, group;
    uint32_t sb_total;   // k / 128
    uint32_t sb_per_split;
    uint32_t splits;
};

template <int BITS>
__global__ __launch_bounds__(256) void qgemv_mfma(QgemvArgs p) {
    extern __shared__ __align__(16) int8_t limbs[];  // [3][m][kslice]
    __shared__ uint32_t max_bits[16];
    __shared__ int exps[16];
    __shared__ int xsum[16 * 64];    // [m][group in split]: sum of X, for the INT4 offset correction
    __shared__ int is_last;

    const int tid = threadIdx.x;
    const int lane = tid % kWave, wave = tid / kWave;
    const uint32_t split = blockIdx.y;
    const uint32_t sb0 = split * p.sb_per_split;
    const uint32_t sb1 = min(sb0 + p.sb_per_split, p.sb_total);
    const uint32_t kslice = p.sb_per_split * 128;
    const uint32_t k0 = sb0 * 128, klen = (sb1 - sb0) * 128;
    const uint32_t g0 = k0 / p.group, gcount = klen / p.group;
    const uint32_t M = p.m;

    // ---- prologue: the activation slice as exact int8 limbs in LDS ----
    if (tid < 16) max_bits[tid] = 0u;
    for (uint32_t i = tid; i < M * gcount; i += 256) xsum[i] = 0;
    __syncthreads();
    for (uint32_t idx = tid; idx < M * klen; idx += 256) {
        const uint32_t m = idx / klen, kk = idx % klen;
        atomicMax(&max_bits[m], __float_as_uint(fabsf(p.a[static_cast<uint64_t>(m) * p.k + k0 + kk])));
    }
    __syncthreads();
    if (tid < 16) {
        int e = 0;
        if (tid < static_cast<int>(M) && max_bits[tid] != 0u) frexpf(__uint_as_float(max_bits[tid]), &e);
        exps[tid] = e;  // max|x| < 2^e
    }
    __syncthreads();
    for (uint32_t idx = tid; idx < M * klen; idx += 256) {
        const uint32_t m = idx / klen, kk = idx % klen;
        const float x = p.a[static_cast<uint64_t>(m) * p.k + k0 + kk];
        const int X = static_cast<int>(rintf(ldexpf(x, 22 - exps[m])));
        const int l0 = ((X + 128) & 255) - 128;
        const int x1 = (X - l0) >> 8;
        const int l1 = ((x1 + 128) & 255) - 128;
        const int l2 = (x1 - l1) >> 8;
        limbs[(0 * M + m) * kslice + kk] = static_cast<int8_t>(l0);
        limbs[(1 * M + m) * kslice + kk] = static_cast<int8_t>(l1);
        limbs[(2 * M + m) * kslice + kk] = static_cast<int8_t>(l2);
        if (BITS == 4) {
            // A wave's 64 consecutive kk share one group (group is a multiple
            // of 64); integer sums keep the correction exact and order-free.
            int sx = X;
#pragma unroll
            for (int off = kWave / 2; off > 0; off >>= 1) sx += __shfl_xor(sx, off, kWave);
            if (lane == 0) atomicAdd(&xsum[m * gcount + kk / p.group], sx);
        }
    }
    __syncthreads();

    // ---- main loop: wave `wave` owns tile nt ----
    const uint32_t nt = blockIdx.x * kWavesPerBlock + wave;
    const uint32_t row = nt * 16 + lane % 16;
    const uint32_t kb4 = lane / 16;
    const uint32_t am = lane % 16;  // A-operand row (activation row)
    const bool a_live = am < M;
    const uint32_t groups_total = p.k / p.group;
    const uint32_t steps_per_group = p.group / 64;
    float total[4] = {0.f, 0.f, 0.f, 0.f};
    const bool tile_live = nt * 16 < p.n;
    if (tile_live) {
        v4i acc0 = {0, 0, 0, 0}, acc1 = acc0, acc2 = acc0;
        const v4i zero = {0, 0, 0, 0};
        uint32_t step = 0;  // 64-k steps since the slice start
        for (uint32_t sb = sb0; sb < sb1; ++sb) {
            uint4 wb[2];
            if (BITS == 4) {
                wb[0] = *reinterpret_cast<const uint4*>(p.tiles + (static_cast<uint64_t>(nt) * p.sb_total + sb) * 1024 +
                                                        lane * 16);
            } else {
                const uint8_t* base = p.tiles + (static_cast<uint64_t>(nt) * p.sb_total + sb) * 2048 + lane * 16;
                wb[0] = *reinterpret_cast<const uint4*>(base);
                wb[1] = *reinterpret_cast<const uint4*>(base + 1024);
            }
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                v4i bv;
                if (BITS == 4) {
                    const uint32_t w0 = s == 0 ? wb[0].x : wb[0].z;
                    const uint32_t w1 = s == 0 ? wb[0].y : wb[0].w;
                    bv[0] = static_cast<int>(w0 & 0x0F0F0F0Fu);
                    bv[1] = static_cast<int>((w0 >> 4) & 0x0F0F0F0Fu);
                    bv[2] = static_cast<int>(w1 & 0x0F0F0F0Fu);
                    bv[3] = static_cast<int>((w1 >> 4) & 0x0F0F0F0Fu);
                } else {
                    bv[0] = static_cast<int>(wb[s].x);
                    bv[1] = static_cast<int>(wb[s].y);
                    bv[2] = static_cast<int>(wb[s].z);
                    bv[3] = static_cast<int>(wb[s].w);
                }
                const uint32_t kl = (sb - sb0) * 128 + s * 64 + kb4 * 16;
                v4i a0 = zero, a1 = zero, a2 = zero;
                if (a_live) {
                    a0 = *reinterpret_cast<const v4i*>(limbs + (0 * M + am) * kslice + kl);
                    a1 = *reinterpret_cast<const v4i*>(limbs + (1 * M + am) * kslice + kl);
                    a2 = *reinterpret_cast<const v4i*>(limbs + (2 * M + am) * kslice + kl);
                }
                acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bv, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bv, acc1, 0, 0, 0);
                acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, bv, acc2, 0, 0, 0);
                ++step;
                if (step % steps_per_group == 0) {
                    const uint32_t gl = step / steps_per_group - 1;  // group within the slice
                    const float sc = row < p.n ? p.scales[static_cast<uint64_t>(row) * groups_total + g0 + gl] : 0.f;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t m = kb4 * 4 + r;
                        float v = fmaf(static_cast<float>(acc2[r]), 65536.0f,
                                       fmaf(static_cast<float>(acc1[r]), 256.0f, static_cast<float>(acc0[r])));
                        if (BITS == 4 && m < M) v -= 8.0f * static_cast<float>(xsum[m * gcount + gl]);
                        total[r] = fmaf(v, sc, total[r]);
                    }
                    acc0 = zero;
                    acc1 = zero;
                    acc2 = zero;
                }
            }
        }
    }

    // ---- results: lane holds rows m = 4*kb4 + r of column `row` ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t m = kb4 * 4 + r;
        if (!tile_live || m >= M || row >= p.n) continue;
        const float v = ldexpf(total[r], exps[m] - 22);
        if (p.splits == 1) p.out[static_cast<uint64_t>(m) * p.n + row] = v;
        else p.partial[(static_cast<uint64_t>(split) * M + m) * p.n + row] = v;
    }
    if (p.splits == 1) return;

    // ---- the last block of this column adds the partials in split order ----
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&p.counters[blockIdx.x], 1u, __ATOMIC_ACQ_REL,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        is_last = prev == p.splits - 1;
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    const uint32_t col0 = blockIdx.x * kWavesPerBlock * 16;
    const uint32_t cols = min(kWavesPerBlock * 16u, p.n - col0);
    for (uint32_t idx = tid; idx < M * cols; idx += 256) {
        const uint32_t m = idx / cols, c = col0 + idx % cols;
        float sum = 0.f;
        for (uint32_t sp = 0; sp < p.splits; ++sp)
            sum += __builtin_nontemporal_load(&p.partial[(static_cast<uint64_t>(sp) * M + m) * p.n + c]);
        p.out[static_cast<uint64_t>(m) * p.n + c] = sum;
    }
    __syncthreads();
    if (tid == 0)
        __hip_atomic_store(&p.counters[blockIdx.x], 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_qgemv_mfma(const float* a, const QuantWeight& w, float* out, uint64_t m, const Workspace& ws,
                             hipStream_t s) {
    if (w.layout != QuantLayout::Mfma || m == 0 || m > 16 || w.k % 128 != 0 || w.group % 64 != 0 ||
        w.group > 64 * 64 || w.n > 0xffffffffull || w.k > 0xffffffffull)
        return hipErrorNotSupported;
    QgemvArgs p;
    p.a = a;
    p.tiles = w.tiles;
    p.scales = w.scales;
    p.out = out;
    p.m = static_cast<uint32_t>(m);
    p.n = static_cast<uint32_t>(w.n);
    p.k = static_cast<uint32_t>(w.k);
    p.group = w.group;
    p.sb_total = p.k / 128;
    const uint32_t n_tiles = (p.n + 15) / 16;
    const uint32_t n_blocks = (n_tiles + kWavesPerBlock - 1) / kWavesPerBlock;

    // Split K so that ~512 blocks run, keeping >= 2 superblocks per split,
    // whole groups per split, and the limb slice within the LDS budget.
    const uint32_t sb_per_group = w.group >= 128 ? w.group / 128 : 1;
    uint32_t splits = (512 + n_blocks - 1) / n_blocks;
    splits = min(splits, max(1u, p.sb_total / 2));
    const uint32_t lds_sb_cap = kLdsLimbBytes / (3 * p.m * 128);
    uint32_t per = (p.sb_total + splits - 1) / splits;
    per = (per + sb_per_group - 1) / sb_per_group * sb_per_group;
    if (per > lds_sb_cap) per = lds_sb_cap / sb_per_group * sb_per_group;
    if (per == 0) return hipErrorNotSupported;
    splits = (p.sb_total + per - 1) / per;
    const uint32_t gcount_max = per * 128 / w.group;
    if (p.m * gcount_max > 16 * 64) return hipErrorNotSupported;
    p.sb_per_split = per;
    p.splits = splits;
    if (splits > 1) {
        const uint64_t need = static_cast<uint64_t>(splits) * p.m * p.n;
        if (need > ws.floats || n_blocks > ws.n_counters) return hipErrorNotSupported;
        p.partial = ws.data;
        p.counters = ws.counters;
    } else {
        p.partial = nullptr;
        p.counters = nullptr;
    }
    const size_t lds = static_cast<size_t>(3) * p.m * per * 128;
    dim3 grid(n_blocks, splits);
    if (w.format == SL_QFORMAT_INT4) qgemv_mfma<4><<<grid, 256, lds, s>>>(p);
    else qgemv_mfma<8><<<grid, 256, lds, s>>>(p);
    return hipGetLastError();
}

}  // namespace slhip
