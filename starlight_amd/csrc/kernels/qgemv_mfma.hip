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
//         codes stored as 4-bit two's complement and arranged so that
//         (w << 4) & 0xF0F0F0F0 and w & 0xF0F0F0F0 give the operand bytes
//         in k order, each the signed byte 16 q; the factor 16 is exact and
//         folded into the final 2^(E-22) scaling.
//   INT8: 2048 bytes, step s at 1024 s, lane l owns bytes [16l, 16l + 16).
// Operand k order within a step: lane l holds k = 16 (l / 16) + j, j < 16,
// for row l % 16 — identical for A and B, which is all the product needs.
//
// Work split: a block of 4 waves owns 4 adjacent 16-row tiles (one per wave)
// and one split of the K superblocks. Every wave issues the loads for all of
// its superblocks (at most kPrefetch) before converting the activations, so
// the whole weight slice is in flight at once — a decode GEMV moves only a
// few MB, about one memory latency's worth, so latency, not bandwidth,
// decides it. K is split until about 1024 waves run; split partials go to the
// workspace and qgemv_reduce adds them in split order (deterministic, and no
// cross-block fence: on this part a device-scope release writes back the
// XCD's L2, which costs far more than one small extra launch).
#include "common.h"
#include "kernels.h"
#include "starlight_hip.h"

namespace slhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWavesPerBlock = 4;
constexpr int kLdsLimbBytes = 48 * 1024;  // 3 limbs x m x k-slice
constexpr int kPrefetch = 8;              // INT4 superblocks in flight per wave (INT8: half)

struct QgemvArgs {
    const float* a;
    const uint8_t* tiles;
    const float* scales;
    float* out;
    float* partial;      // [splits, m, n] when splits > 1
    uint32_t m, n, k, group;
    uint32_t sb_total;   // k / 128
    uint32_t sb_per_split;
    uint32_t splits;
};

template <int BITS>
__global__ __launch_bounds__(256) void qgemv_mfma(QgemvArgs p) {
    prefetch_kernarg<arg_bytes<QgemvArgs>()>();
    constexpr int PF = BITS == 4 ? kPrefetch : kPrefetch / 2;  // superblocks in flight per wave
    extern __shared__ __align__(16) int8_t limbs[];  // [3][m][kslice]
    __shared__ uint32_t max_bits[16];
    __shared__ int exps[16];

    const int tid = threadIdx.x;
    const int lane = tid % kWave, wave = tid / kWave;
    const uint32_t split = blockIdx.y;
    const uint32_t sb0 = split * p.sb_per_split;
    const uint32_t sb1 = min(sb0 + p.sb_per_split, p.sb_total);
    const uint32_t kslice = p.sb_per_split * 128;
    const uint32_t k0 = sb0 * 128, klen = (sb1 - sb0) * 128;
    const uint32_t g0 = k0 / p.group;
    const uint32_t M = p.m;

    // ---- the wave's weight stream: a rolling window of kPrefetch
    // superblocks in registers, started before the prologue so the first
    // HBM round trip overlaps the activation conversion ----
    const uint32_t nt = blockIdx.x * kWavesPerBlock + wave;
    const bool tile_live = nt * 16 < p.n;
    const uint8_t* wtile = p.tiles + static_cast<uint64_t>(nt) * p.sb_total * (BITS == 4 ? 1024 : 2048) + lane * 16;
    uint4 w0[PF], w1[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) {
        const uint32_t sb = sb0 + i;
        if (tile_live && sb < sb1) {
            if constexpr (BITS == 4) {
                w0[i] = *reinterpret_cast<const uint4*>(wtile + static_cast<uint64_t>(sb) * 1024);
            } else {
                w0[i] = *reinterpret_cast<const uint4*>(wtile + static_cast<uint64_t>(sb) * 2048);
                w1[i] = *reinterpret_cast<const uint4*>(wtile + static_cast<uint64_t>(sb) * 2048 + 1024);
            }
        }
    }

    // ---- prologue: the activation slice as exact int8 limbs in LDS ----
    // (float4 loads, four in flight per thread per pass)
    if (tid < 16) max_bits[tid] = 0u;
    __syncthreads();
    const uint32_t q4 = klen / 4;  // float4 per row slice
    for (uint32_t m = 0; m < M; ++m) {
        const float4* xr = reinterpret_cast<const float4*>(p.a + static_cast<uint64_t>(m) * p.k + k0);
        float mx = 0.f;
        for (uint32_t f = tid; f < q4; f += 1024) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = f + 256 * u < q4 ? xr[f + 256 * u] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
        }
        mx = wave_max(mx);
        if (lane == 0) atomicMax(&max_bits[m], __float_as_uint(mx));
    }
    __syncthreads();
    if (tid < 16) {
        int e = 0;
        if (tid < static_cast<int>(M) && max_bits[tid] != 0u) frexpf(__uint_as_float(max_bits[tid]), &e);
        exps[tid] = e;  // max|x| < 2^e
    }
    __syncthreads();
    for (uint32_t m = 0; m < M; ++m) {
        const float4* xr = reinterpret_cast<const float4*>(p.a + static_cast<uint64_t>(m) * p.k + k0);
        const int shift = 22 - exps[m];
        for (uint32_t f0 = 0; f0 < q4; f0 += 1024) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t f = f0 + tid + 256 * u;
                v[u] = f < q4 ? xr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t f = f0 + tid + 256 * u;
                if (f0 + (tid & ~(kWave - 1)) + 256 * u >= q4) continue;  // whole wave out of range
                const float xe[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
                uint32_t packed[3] = {0u, 0u, 0u};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int X = f < q4 ? static_cast<int>(rintf(ldexpf(xe[e], shift))) : 0;
                    const int l0 = ((X + 128) & 255) - 128;
                    const int x1 = (X - l0) >> 8;
                    const int l1 = ((x1 + 128) & 255) - 128;
                    const int l2 = (x1 - l1) >> 8;
                    packed[0] |= (static_cast<uint32_t>(l0) & 0xFFu) << (8 * e);
                    packed[1] |= (static_cast<uint32_t>(l1) & 0xFFu) << (8 * e);
                    packed[2] |= (static_cast<uint32_t>(l2) & 0xFFu) << (8 * e);
                }
                if (f < q4) {
#pragma unroll
                    for (int limb = 0; limb < 3; ++limb)
                        *reinterpret_cast<uint32_t*>(limbs + (limb * M + m) * kslice + 4 * f) = packed[limb];
                }
            }
        }
    }
    __syncthreads();

    // ---- main loop: wave `wave` owns tile nt ----
    const uint32_t row = nt * 16 + lane % 16;
    const uint32_t kb4 = lane / 16;
    const uint32_t am = lane % 16;  // A-operand row (activation row)
    const bool a_live = am < M;
    const uint32_t groups_total = p.k / p.group;
    const uint32_t steps_per_group = p.group / 64;
    float total[4] = {0.f, 0.f, 0.f, 0.f};
    if (tile_live) {
        v4i acc0 = {0, 0, 0, 0}, acc1 = acc0, acc2 = acc0;
        const v4i zero = {0, 0, 0, 0};
        uint32_t step = 0;  // 64-k steps since the slice start
        for (uint32_t base = sb0; base < sb1; base += PF) {
#pragma unroll
            for (int i = 0; i < PF; ++i) {
                const uint32_t sb = base + i;
                if (sb >= sb1) break;
                const uint4 c0 = w0[i];
                uint4 c1 = c0;
                if constexpr (BITS == 8) c1 = w1[i];
                const uint32_t nsb = sb + PF;
                if (nsb < sb1) {
                    if constexpr (BITS == 4) {
                        w0[i] = *reinterpret_cast<const uint4*>(wtile + static_cast<uint64_t>(nsb) * 1024);
                    } else {
                        w0[i] = *reinterpret_cast<const uint4*>(wtile + static_cast<uint64_t>(nsb) * 2048);
                        w1[i] = *reinterpret_cast<const uint4*>(wtile + static_cast<uint64_t>(nsb) * 2048 + 1024);
                    }
                }
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    v4i bv;
                    if (BITS == 4) {
                        const uint32_t wa = s == 0 ? c0.x : c0.z;
                        const uint32_t wb = s == 0 ? c0.y : c0.w;
                        bv[0] = static_cast<int>((wa << 4) & 0xF0F0F0F0u);
                        bv[1] = static_cast<int>(wa & 0xF0F0F0F0u);
                        bv[2] = static_cast<int>((wb << 4) & 0xF0F0F0F0u);
                        bv[3] = static_cast<int>(wb & 0xF0F0F0F0u);
                    } else {
                        const uint4 cw = s == 0 ? c0 : c1;
                        bv[0] = static_cast<int>(cw.x);
                        bv[1] = static_cast<int>(cw.y);
                        bv[2] = static_cast<int>(cw.z);
                        bv[3] = static_cast<int>(cw.w);
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
                        const float sc =
                            row < p.n ? p.scales[static_cast<uint64_t>(row) * groups_total + g0 + gl] : 0.f;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float v = fmaf(static_cast<float>(acc2[r]), 65536.0f,
                                           fmaf(static_cast<float>(acc1[r]), 256.0f, static_cast<float>(acc0[r])));
                            total[r] = fmaf(v, sc, total[r]);
                        }
                        acc0 = zero;
                        acc1 = zero;
                        acc2 = zero;
                    }
                }
            }
        }
    }

    // ---- results: lane holds rows m = 4*kb4 + r of column `row` ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t m = kb4 * 4 + r;
        if (!tile_live || m >= M || row >= p.n) continue;
        const float v = ldexpf(total[r], exps[m] - 22 - (BITS == 4 ? 4 : 0));  // INT4 operands are 16 q
        if (p.splits == 1) p.out[static_cast<uint64_t>(m) * p.n + row] = v;
        else p.partial[(static_cast<uint64_t>(split) * M + m) * p.n + row] = v;
    }
}

// out[i] = sum over splits (in order) of partial[split][i], i < m * n.
__global__ __launch_bounds__(256) void qgemv_reduce(const float* __restrict__ partial, float* __restrict__ out,
                                                    uint64_t count, uint32_t splits) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        float sum = 0.f;
        for (uint32_t sp = 0; sp < splits; ++sp) sum += partial[sp * count + i];
        out[i] = sum;
    }
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

    // Split K so that each wave holds at most kPrefetch superblocks (INT8:
    // half, two loads each), about 1024 waves run, splits cover whole
    // groups, and the limb slice fits the LDS budget.
    const uint32_t sb_per_group = w.group >= 128 ? w.group / 128 : 1;
    const uint32_t pf = w.format == SL_QFORMAT_INT4 ? kPrefetch : kPrefetch / 2;  // PF of the kernel
    const uint32_t lds_sb_cap = kLdsLimbBytes / (3 * p.m * 128);
    uint32_t per_cap = min(pf, lds_sb_cap) / sb_per_group * sb_per_group;
    if (per_cap == 0) return hipErrorNotSupported;
    uint32_t splits = max((p.sb_total + per_cap - 1) / per_cap, (1024 + n_tiles - 1) / n_tiles);
    splits = min(splits, p.sb_total / sb_per_group);
    uint32_t per = (p.sb_total + splits - 1) / splits;
    per = (per + sb_per_group - 1) / sb_per_group * sb_per_group;
    if (per > per_cap) per = per_cap;
    splits = (p.sb_total + per - 1) / per;
    if (p.m * (per * 128 / w.group) > 16 * 64) return hipErrorNotSupported;
    p.sb_per_split = per;
    p.splits = splits;
    if (splits > 1) {
        const uint64_t need = static_cast<uint64_t>(splits) * p.m * p.n;
        if (need > ws.floats) return hipErrorNotSupported;
        p.partial = ws.data;
    } else {
        p.partial = nullptr;
    }
    const size_t lds = static_cast<size_t>(3) * p.m * per * 128;
    dim3 grid(n_blocks, splits);
    if (w.format == SL_QFORMAT_INT4) qgemv_mfma<4><<<grid, 256, lds, s>>>(p);
    else qgemv_mfma<8><<<grid, 256, lds, s>>>(p);
    if (splits > 1) {
        const uint64_t count = static_cast<uint64_t>(p.m) * p.n;
        qgemv_reduce<<<grid_for(count, 256, 1024), 256, 0, s>>>(p.partial, out, count, splits);
    }
    return hipGetLastError();
}

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_qgemv_mfma() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&qgemv_reduce));
}

}  // namespace slhip
