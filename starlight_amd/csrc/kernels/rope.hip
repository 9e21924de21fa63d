// Rope (reference/rope.rs:32-141), written out of place (the device copies
// nothing first: out = rotate(x)).
//
// One thread per (batch, token, pair): it computes the angle
// position / theta^(2*pair/head_dim), its sine and cosine in f64 exactly where
// the reference does, rounds them to f32 once, and then rotates that pair in
// every head, so the f64 work is shared across heads. Lanes run over
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

}  // namespace

hipError_t launch_rope(const float* x, const uint32_t* positions, float* out, uint64_t batch,
                       uint64_t heads, uint64_t seq, uint64_t head_dim, float theta, bool interleaved,
                       hipStream_t s) {
    const uint64_t tokens = batch * seq;
    if (tokens == 0 || heads == 0 || head_dim == 0) return hipSuccess;
    if (tokens > 0x7fffffffull || heads * head_dim > 0xffffffffull) return hipErrorInvalidValue;
    const size_t lds = head_dim * sizeof(float);
    const unsigned grid = static_cast<unsigned>(tokens);
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

}  // namespace slhip
