// Rope (reference/rope.rs:32-141), written out of place (the device copies
// nothing first: out = rotate(x)).
//
// One block per (batch, token): it computes the angles
// position / theta^(2*pair/head_dim), their sine and cosine in f64 exactly
// where the reference does, rounds them to f32 once, and then rotates those
// pairs in every head, so the f64 work is shared across heads. Lanes run over
// consecutive pairs, so each head's loads and stores are contiguous. The
// rotation is x*c - y*s, x*s + y*c in f32 with no contraction (the file is
// built with -ffp-contract=off), matching the reference bit for bit whenever
// the device's f64 pow/sin/cos round to the same f32 as the host libm.
#include "common.h"
#include "kernels.h"

namespace slhip {
namespace {

// One block per (batch, token): the first head_dim/2 threads compute the
// pair angles' sine and cosine once (f64, as rope.rs:32-35, 72-75), then the
// whole block rotates that token's pairs in every head, each thread issuing
// all of its loads before its stores.
template <bool INTERLEAVED>
__global__ __launch_bounds__(256) void rope_kernel(const float* __restrict__ x, const uint32_t* __restrict__ pos,
                                                   float* __restrict__ out, uint32_t heads, uint32_t seq,
                                                   uint32_t head_dim, double theta) {
    prefetch_kernarg<arg_bytes<const float*, const uint32_t*, float*, uint32_t, uint32_t, uint32_t, double>()>();
    extern __shared__ float sc[];  // [half] sine, [half] cosine
    const uint32_t half = head_dim / 2;
    const uint64_t bt = blockIdx.x;  // b * seq + t
    const uint64_t b = bt / seq, t = bt % seq;
    const double position = static_cast<double>(pos[bt]);
    for (uint32_t pair = threadIdx.x; pair < half; pair += blockDim.x) {
        const double exponent = 2.0 * static_cast<double>(pair) / static_cast<double>(head_dim);
        const double angle = position / pow(theta, exponent);
        sc[pair] = static_cast<float>(sin(angle));
        sc[half + pair] = static_cast<float>(cos(angle));
    }
    __syncthreads();
    const uint32_t total = heads * half;
    for (uint32_t i0 = threadIdx.x; i0 < total; i0 += 4 * blockDim.x) {
        float first[4], second[4];
        uint64_t idx0[4], idx1[4];
        uint32_t pr[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t i = i0 + u * blockDim.x;
            const uint32_t h = i / half, pair = i % half;
            pr[u] = pair;
            const uint64_t base = ((b * heads + h) * seq + t) * head_dim;
            idx0[u] = base + (INTERLEAVED ? 2 * pair : pair);
            idx1[u] = base + (INTERLEAVED ? 2 * pair + 1 : pair + half);
            if (i < total) {
                first[u] = x[idx0[u]];
                second[u] = x[idx1[u]];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t i = i0 + u * blockDim.x;
            if (i >= total) continue;
            const float sine = sc[pr[u]], cosine = sc[half + pr[u]];
            stream_store(out + idx0[u], first[u] * cosine - second[u] * sine);
            stream_store(out + idx1[u], first[u] * sine + second[u] * cosine);
        }
    }
}

// The same rotation with 16-byte accesses, for head_dim % 8 == 0 and 16-byte
// aligned x and out. An item is one float4 of pairs: NeoX pairs 4c .. 4c+3
// of a head (the float4 at 4c and the one at half + 4c), GPT-J pairs 2c and
// 2c+1 (the float4 at 4c). Each thread issues the loads of its first kIpt
// items before the block works out the sine and cosine table, so the f64
// work overlaps the memory round trip.
constexpr int kRopeIpt = 4;

template <bool INTERLEAVED>
__global__ __launch_bounds__(256) void rope_vec4(const float4* __restrict__ x, const uint32_t* __restrict__ pos,
                                                 float4* __restrict__ out, uint32_t heads, uint32_t seq,
                                                 uint32_t head_dim, double theta) {
    prefetch_kernarg<arg_bytes<const float4*, const uint32_t*, float4*, uint32_t, uint32_t, uint32_t, double>()>();
    extern __shared__ float sc[];  // [half] sine, [half] cosine
    const uint32_t half = head_dim / 2, d4 = head_dim / 4;
    const uint32_t per_head = INTERLEAVED ? d4 : d4 / 2;  // items per head
    const uint32_t total = heads * per_head;
    const uint64_t bt = blockIdx.x;  // b * seq + t
    const uint64_t b = bt / seq, t = bt % seq;
    // float4 index of item i's first operand
    auto at = [&](uint32_t i) -> uint64_t {
        const uint32_t h = i / per_head, c = i % per_head;
        return ((b * heads + h) * seq + t) * d4 + c;
    };
    float4 v0[kRopeIpt], v1[kRopeIpt];
    auto load = [&](uint32_t i0) {
#pragma unroll
        for (int u = 0; u < kRopeIpt; ++u) {
            const uint32_t i = i0 + u * blockDim.x;
            if (i < total) {
                v0[u] = x[at(i)];
                if (!INTERLEAVED) v1[u] = x[at(i) + d4 / 2];
            }
        }
    };
    auto rotate_store = [&](uint32_t i0) {
#pragma unroll
        for (int u = 0; u < kRopeIpt; ++u) {
            const uint32_t i = i0 + u * blockDim.x;
            if (i >= total) continue;
            const uint32_t c = i % per_head;
            if constexpr (INTERLEAVED) {
                // pairs (x, y) and (z, w): 2c and 2c + 1
                const float s0 = sc[2 * c], c0 = sc[half + 2 * c], s1 = sc[2 * c + 1], c1 = sc[half + 2 * c + 1];
                const float4 a = v0[u];
                stream_store(out + at(i), make_float4(a.x * c0 - a.y * s0, a.x * s0 + a.y * c0, a.z * c1 - a.w * s1,
                                                      a.z * s1 + a.w * c1));
            } else {
                const float4 a = v0[u], e = v1[u];
                const uint32_t p0 = 4 * c;
                const float s0 = sc[p0], s1 = sc[p0 + 1], s2 = sc[p0 + 2], s3 = sc[p0 + 3];
                const float c0 = sc[half + p0], c1 = sc[half + p0 + 1], c2 = sc[half + p0 + 2],
                            c3 = sc[half + p0 + 3];
                stream_store(out + at(i), make_float4(a.x * c0 - e.x * s0, a.y * c1 - e.y * s1, a.z * c2 - e.z * s2,
                                                      a.w * c3 - e.w * s3));
                stream_store(out + at(i) + d4 / 2, make_float4(a.x * s0 + e.x * c0, a.y * s1 + e.y * c1,
                                                               a.z * s2 + e.z * c2, a.w * s3 + e.w * c3));
            }
        }
    };
    // first round's loads, then the table (every thread, while they are in
    // flight), one barrier, then the rounds
    load(threadIdx.x);
    const double position = static_cast<double>(pos[bt]);
    for (uint32_t pair = threadIdx.x; pair < half; pair += blockDim.x) {
        const double exponent = 2.0 * static_cast<double>(pair) / static_cast<double>(head_dim);
        const double angle = position / pow(theta, exponent);
        sc[pair] = static_cast<float>(sin(angle));
        sc[half + pair] = static_cast<float>(cos(angle));
    }
    __syncthreads();
    rotate_store(threadIdx.x);
    for (uint32_t i0 = threadIdx.x + kRopeIpt * blockDim.x; i0 < total; i0 += kRopeIpt * blockDim.x) {
        load(i0);
        rotate_store(i0);
    }
}

}  // namespace

hipError_t launch_rope(const float* x, const uint32_t* positions, float* out, uint64_t batch,
                       uint64_t heads, uint64_t seq, uint64_t head_dim, float theta, bool interleaved,
                       hipStream_t s) {
    const uint64_t tokens = batch * seq;
    if (tokens == 0 || heads == 0 || head_dim == 0) return hipSuccess;
    if (tokens > 0x7fffffffull || heads * head_dim > 0xffffffffull) return hipErrorInvalidValue;
    const size_t lds = head_dim * sizeof(float);
    const unsigned grid = static_cast<unsigned>(tokens);
    if (head_dim % 8 == 0 && aligned16(x) && aligned16(out)) {
        const float4* x4 = reinterpret_cast<const float4*>(x);
        float4* o4 = reinterpret_cast<float4*>(out);
        if (interleaved)
            rope_vec4<true><<<grid, 256, lds, s>>>(x4, positions, o4, static_cast<uint32_t>(heads),
                                                   static_cast<uint32_t>(seq), static_cast<uint32_t>(head_dim),
                                                   static_cast<double>(theta));
        else
            rope_vec4<false><<<grid, 256, lds, s>>>(x4, positions, o4, static_cast<uint32_t>(heads),
                                                    static_cast<uint32_t>(seq), static_cast<uint32_t>(head_dim),
                                                    static_cast<double>(theta));
        return hipGetLastError();
    }
    if (interleaved)
        rope_kernel<true><<<grid, 256, lds, s>>>(x, positions, out, static_cast<uint32_t>(heads),
                                                 static_cast<uint32_t>(seq), static_cast<uint32_t>(head_dim),
                                                 static_cast<double>(theta));
    else
        rope_kernel<false><<<grid, 256, lds, s>>>(x, positions, out, static_cast<uint32_t>(heads),
                                                  static_cast<uint32_t>(seq), static_cast<uint32_t>(head_dim),
                                                  static_cast<double>(theta));
    return hipGetLastError();
}

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_rope() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&rope_kernel<false>));
}

}  // namespace slhip
