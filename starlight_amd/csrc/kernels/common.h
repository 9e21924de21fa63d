// Shared device helpers for the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slhip {

constexpr int kWave = 64;

// Cross-lane reductions on the DPP network: within each 16-lane row,
// xor 1 and xor 2 (quad_perm), then the half-row and row mirrors, leave the
// row's total in every lane of the row (the same bits in each, the
// operations being commutative); readlane then combines the four rows into
// a wave-uniform value. No LDS round trips, unlike ds_bpermute shuffles.
// All 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppRowRor8 = 0x128;  // row_ror:8, lane i of a 16-lane row takes lane (i + 8) % 16

__device__ __forceinline__ float row_sum(float v) {
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppHalfMirror>(v);
    v += dpp_f<kDppMirror>(v);
    return v;
}
__device__ __forceinline__ int row_sum(int v) {
    v += dpp_i<kDppXor1>(v);
    v += dpp_i<kDppXor2>(v);
    v += dpp_i<kDppHalfMirror>(v);
    v += dpp_i<kDppMirror>(v);
    return v;
}
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    return v;
}
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
    const float r = row_sum(v);
    return (lane_value(r, 0) + lane_value(r, 16)) + (lane_value(r, 32) + lane_value(r, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    const float r = row_max(v);
    return fmaxf(fmaxf(lane_value(r, 0), lane_value(r, 16)), fmaxf(lane_value(r, 32), lane_value(r, 48)));
}

// The largest v of the wave, for values ordered as unsigned integers (such
// as the bit patterns of non-negative floats): one DPP max per step within
// the rows (a float max would first quiet each operand), then the four rows
// in scalar registers.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, static_cast<uint32_t>(dpp_i<kDppXor1>(static_cast<int>(v))));
    v = max(v, static_cast<uint32_t>(dpp_i<kDppXor2>(static_cast<int>(v))));
    v = max(v, static_cast<uint32_t>(dpp_i<kDppHalfMirror>(static_cast<int>(v))));
    v = max(v, static_cast<uint32_t>(dpp_i<kDppMirror>(static_cast<int>(v))));
    const uint32_t a = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0));
    const uint32_t b = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16));
    const uint32_t c = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32));
    const uint32_t d = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 48));
    // (each pair's max kept scalar: a three-input max would go to the VALU)
    const uint32_t ab = __builtin_amdgcn_readfirstlane(max(a, b));
    const uint32_t cd = __builtin_amdgcn_readfirstlane(max(c, d));
    return max(ab, cd);
}

// Block-wide sum/max for blocks of up to 1024 threads; every thread gets the
// result. `scratch` needs blockDim.x / 64 floats of LDS.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int waves = (blockDim.x + kWave - 1) / kWave;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float total = 0.f;
    for (int i = 0; i < waves; ++i) total += scratch[i];
    return total;
}

__device__ __forceinline__ float block_max(float v, float* scratch) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int waves = (blockDim.x + kWave - 1) / kWave;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float m = -INFINITY;
    for (int i = 0; i < waves; ++i) m = fmaxf(m, scratch[i]);
    return m;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Stores of outputs that are written once and read by a later launch, with
// the non-temporal hint: streamed past the caches, which lifts the write
// bandwidth of large row-wise kernels (a float4 copy of 2 x 64 MiB: about
// 5.6 TB/s with plain stores, 6.7 TB/s with these, on MI355X).
typedef float sl_v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void stream_store(float4* p, float4 v) {
    __builtin_nontemporal_store(sl_v4f{v.x, v.y, v.z, v.w}, reinterpret_cast<sl_v4f*>(p));
}
__device__ __forceinline__ void stream_store(float* p, float v) { __builtin_nontemporal_store(v, p); }

// v from lane i ^ 16 and i ^ 32 of the wave, with the gfx950 lane swaps:
// VALU operations, where a ds_bpermute shuffle is an LDS round trip. With
// both operands v, v_permlane16_swap leaves the even 16-lane rows of its
// first result and the odd rows of its second unchanged, the other rows
// taking their neighbour's values; v_permlane32_swap does the same for the
// two 32-lane halves.
__device__ __forceinline__ float lane_xor16(float v) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 16) ? s[0] : s[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 32) ? s[0] : s[1]);
}

// N wave reductions at once (N = 2, 4 or 8 values per lane, as bit
// patterns; OP combines two, commutatively). Each level of a butterfly
// pairs two of a lane's values and exchanges half of them: at distance 32,
// v_permlane32_swap(a, b) leaves a's lower half with b's lower half, and b
// with both upper halves, so one combine of the two results reduces a in
// the lower lanes and b in the upper ones; at distance 16 v_permlane16_swap
// does the same for 16-lane rows; at distance 8 a DPP row rotate by 8. The
// one value left is then reduced within groups of 64 / N lanes on the DPP
// network. Lane l ends with the total of value l / (64 / N), every lane of a
// group holding the same bits. For N = 8 that is 7 exchanges (4 + 2 + 1)
// and 3 DPP steps, against 8 separate reductions of 4 DPP steps and 4
// readlanes each. All 64 lanes must be active.
template <int N, typename Op>
__device__ __forceinline__ uint32_t lane_reduce_bits(const uint32_t (&v)[N], Op op) {
    static_assert(N == 2 || N == 4 || N == 8, "two, four or eight values per lane");
    uint32_t b[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {  // pairs (i, i + N / 2): lanes 0-31 keep i, 32-63 i + N / 2
        const auto s = __builtin_amdgcn_permlane32_swap(v[i], v[i + N / 2], false, false);
        b[i] = op(s[0], s[1]);
    }
    uint32_t r;
    if constexpr (N == 2) {
        r = b[0];
    } else {
        uint32_t c[N / 4];
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {  // 16-lane rows 0, 1, 2, 3 keep slots i, i + N / 4 (lower, upper)
            const auto s = __builtin_amdgcn_permlane16_swap(b[i], b[i + N / 4], false, false);
            c[i] = op(s[0], s[1]);
        }
        if constexpr (N == 4) {
            r = c[0];
        } else {  // the 8-lane halves of each row keep c[0] and c[1]
            const bool upper = (threadIdx.x & 8) != 0;
            const uint32_t keep = upper ? c[1] : c[0], give = upper ? c[0] : c[1];
            r = op(keep, static_cast<uint32_t>(dpp_i<kDppRowRor8>(static_cast<int>(give))));
        }
    }
    r = op(r, static_cast<uint32_t>(dpp_i<kDppXor1>(static_cast<int>(r))));
    r = op(r, static_cast<uint32_t>(dpp_i<kDppXor2>(static_cast<int>(r))));
    r = op(r, static_cast<uint32_t>(dpp_i<kDppHalfMirror>(static_cast<int>(r))));
    if constexpr (N <= 4) r = op(r, static_cast<uint32_t>(dpp_i<kDppMirror>(static_cast<int>(r))));
    if constexpr (N == 2) {
        const auto s = __builtin_amdgcn_permlane16_swap(r, r, false, false);
        r = op(r, (threadIdx.x & 16) ? s[0] : s[1]);
    }
    return r;
}
template <int N>
__device__ __forceinline__ float lane_reduce_sum(const float (&v)[N]) {
    uint32_t bits[N];
#pragma unroll
    for (int i = 0; i < N; ++i) bits[i] = __float_as_uint(v[i]);
    return __uint_as_float(lane_reduce_bits<N>(
        bits, [](uint32_t a, uint32_t b) { return __float_as_uint(__uint_as_float(a) + __uint_as_float(b)); }));
}
template <int N>
__device__ __forceinline__ uint32_t lane_reduce_max_u32(const uint32_t (&v)[N]) {
    return lane_reduce_bits<N>(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}

// Pulls the first BYTES of the kernel's argument segment into the scalar
// cache with one batch of independent loads (one word per 64-byte line) and
// waits for them once. Left to itself the compiler fetches arguments as
// control flow needs them, and each batch that touches a new line costs a
// memory round trip (about 0.6 us) before the kernel's first global load.
// BYTES is the explicit arguments' size (arg_bytes below); the last word
// is touched too, so the lines are covered whatever the segment's alignment.
// Kernels whose explicit arguments are all scalars or pointers, at most
// six, do not call it: the library is built to preload up to six leading
// such arguments into scalar registers, so they have nothing to fetch.
template <uint32_t BYTES>
__device__ __forceinline__ void prefetch_kernarg() {
    static_assert(BYTES >= 4, "no arguments to fetch");
    typedef __attribute__((address_space(4))) uint32_t ka_word;
    const ka_word* ka = (const ka_word*)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t t = ka[((BYTES - 1) & ~3u) / 4];
#pragma unroll
    for (uint32_t o = 0; o < BYTES; o += 64) t += ka[o / 4];
    asm volatile("; kernarg lines loaded %0, %1 bytes" ::"s"(t), "i"(BYTES));
}

// Size of a kernel's explicit arguments of types T...: each argument at its
// natural alignment, in order.
template <typename... T>
constexpr uint32_t arg_bytes() {
    uint32_t off = 0;
    ((off = static_cast<uint32_t>((off + alignof(T) - 1) / alignof(T) * alignof(T) + sizeof(T))), ...);
    return off;
}

// Compute units of the current device (all devices of a process are taken
// to be the same part).
inline unsigned compute_units() {
    static unsigned cus = 0;
    if (cus == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = static_cast<unsigned>(v);
        else
            cus = 256;
    }
    return cus;
}

// Largest LDS allocation one workgroup may make on the current device.
inline size_t max_lds_per_block() {
    static size_t bytes = 0;
    if (bytes == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0)
            bytes = static_cast<size_t>(v);
        else
            bytes = 64 * 1024;
    }
    return bytes;
}

inline unsigned grid_for(uint64_t work, unsigned per_block, unsigned cap) {
    uint64_t g = (work + per_block - 1) / per_block;
    if (g == 0) g = 1;
    return static_cast<unsigned>(g < cap ? g : cap);
}

}  // namespace slhip
