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

template <bool INTERLEAVED>
__global__ __launch_bounds__(256) void rope_kernel(const float* __restrict__ x, const uint32_t* __restrict__ pos,
                                                   float* __restrict__ out, uint64_t batch, uint64_t heads,
                                                   uint64_t seq, uint64_t head_dim, double theta) {
    const uint64_t half = head_dim / 2;
    const uint64_t total = batch * seq * half;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        const uint64_t pair = i % half;
        const uint64_t bt = i / half;  // b * seq + t
        const uint64_t b = bt / seq, t = bt % seq;
        const double position = static_cast<double>(pos[bt]);
        const double exponent = 2.0 * static_cast<double>(pair) / static_cast<double>(head_dim);
        const double angle = position / pow(theta, exponent);
        const float sine = static_cast<float>(sin(angle));
        const float cosine = static_cast<float>(cos(angle));
        const uint64_t i0 = INTERLEAVED ? 2 * pair : pair;
        const uint64_t i1 = INTERLEAVED ? 2 * pair + 1 : pair + half;
        for (uint64_t h = 0; h < heads; ++h) {
            const uint64_t base = ((b * heads + h) * seq + t) * head_dim;
            const float first = x[base + i0];
            const float second = x[base + i1];
            out[base + i0] = first * cosine - second * sine;
            out[base + i1] = first * sine + second * cosine;
        }
    }
}

}  // namespace

hipError_t launch_rope(const float* x, const uint32_t* positions, float* out, uint64_t batch,
                       uint64_t heads, uint64_t seq, uint64_t head_dim, float theta, bool interleaved,
                       hipStream_t s) {
    const uint64_t total = batch * seq * (head_dim / 2);
    if (total == 0 || heads == 0) return hipSuccess;
    const unsigned grid = grid_for(total, 256, 256 * 16);
    if (interleaved)
        rope_kernel<true><<<grid, 256, 0, s>>>(x, positions, out, batch, heads, seq, head_dim,
                                               static_cast<double>(theta));
    else
        rope_kernel<false><<<grid, 256, 0, s>>>(x, positions, out, batch, heads, seq, head_dim,
                                                static_cast<double>(theta));
    return hipGetLastError();
}

}  // namespace slhip
