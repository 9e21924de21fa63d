// RmsNorm (reference/norm.rs:27-60) and Softmax / SoftmaxCausal
// (reference/softmax.rs:19-114): one workgroup per row.
//
// A row lives in registers between the reduction and the write-back, so HBM
// sees each input element read once and each output written once. The
// reduction runs per wave with xor-shuffles, then across the block's waves in
// LDS. Per-row arithmetic keeps the reference's formulas: inv = 1/sqrt(ss/H +
// eps) computed once, out = (x * inv) * w; softmax subtracts the row max,
// exponentiates with the precise expf and multiplies by 1/sum.
#include "common.h"
#include "kernels.h"

namespace slhip {
namespace {

// RMSNorm with the row held in VPT float4 per thread (hidden <= 4*VPT*256).
template <int VPT>
__global__ __launch_bounds__(256) void rms_norm_vec(const float4* __restrict__ x, const float4* __restrict__ w,
                                                    float4* __restrict__ out, uint32_t hidden4, float hidden_f,
                                                    float eps) {
    __shared__ float scratch[4];
    const uint64_t row = blockIdx.x;
    const float4* xr = x + row * hidden4;
    float4 v[VPT], g[VPT];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t c = threadIdx.x + i * 256u;
        v[i] = c < hidden4 ? xr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // the weight row goes out with the input, not after the reduction
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t c = threadIdx.x + i * 256u;
        g[i] = c < hidden4 ? w[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        ss = fmaf(v[i].x, v[i].x, ss);
        ss = fmaf(v[i].y, v[i].y, ss);
        ss = fmaf(v[i].z, v[i].z, ss);
        ss = fmaf(v[i].w, v[i].w, ss);
    }
    ss = block_sum(ss, scratch);
    const float inv = 1.0f / sqrtf(ss / hidden_f + eps);
    float4* orow = out + row * hidden4;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t c = threadIdx.x + i * 256u;
        if (c < hidden4) {
            float4 r;
            r.x = (v[i].x * inv) * g[i].x;
            r.y = (v[i].y * inv) * g[i].y;
            r.z = (v[i].z * inv) * g[i].z;
            r.w = (v[i].w * inv) * g[i].w;
            stream_store(orow + c, r);
        }
    }
}

// General RMSNorm: any hidden size and alignment, two passes over the row.
__global__ __launch_bounds__(256) void rms_norm_any(const float* __restrict__ x, const float* __restrict__ w,
                                                    float* __restrict__ out, uint64_t hidden, float eps) {
    __shared__ float scratch[4];
    const float* xr = x + blockIdx.x * hidden;
    float ss = 0.f;
    for (uint64_t c = threadIdx.x; c < hidden; c += 256) ss = fmaf(xr[c], xr[c], ss);
    ss = block_sum(ss, scratch);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(hidden) + eps);
    float* orow = out + blockIdx.x * hidden;
    for (uint64_t c = threadIdx.x; c < hidden; c += 256) orow[c] = (xr[c] * inv) * w[c];
}

// Softmax with the row in registers: up to 256 * VPT columns.
template <int VPT, bool CAUSAL>
__global__ __launch_bounds__(256) void softmax_regs(const float* __restrict__ x, float* __restrict__ out,
                                                    uint32_t cols, uint32_t seq, uint32_t past_len,
                                                    const uint32_t* __restrict__ dyn) {
    __shared__ float scratch[4];
    const uint64_t row = blockIdx.x;
    if (CAUSAL && dyn != nullptr) past_len = dyn[0];
    const uint32_t visible = CAUSAL ? past_len + static_cast<uint32_t>(row % seq) + 1u : cols;
    const float* xr = x + row * cols;
    float v[VPT];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t c = threadIdx.x + i * 256u;
        v[i] = c < visible ? xr[c] : -INFINITY;
        m = fmaxf(m, v[i]);
    }
    m = block_max(m, scratch);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t c = threadIdx.x + i * 256u;
        v[i] = c < visible ? expf(v[i] - m) : 0.f;
        sum += v[i];
    }
    sum = block_sum(sum, scratch);
    const float inv = 1.0f / sum;
    float* orow = out + row * cols;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t c = threadIdx.x + i * 256u;
        if (c < cols) stream_store(orow + c, v[i] * inv);  // masked columns: exactly 0
    }
}

// General softmax: three passes over the row for very wide rows.
template <bool CAUSAL>
__global__ __launch_bounds__(256) void softmax_any(const float* __restrict__ x, float* __restrict__ out,
                                                   uint64_t cols, uint64_t seq, uint64_t past_len,
                                                   const uint32_t* __restrict__ dyn) {
    __shared__ float scratch[4];
    const uint64_t row = blockIdx.x;
    if (CAUSAL && dyn != nullptr) past_len = dyn[0];
    const uint64_t visible = CAUSAL ? past_len + row % seq + 1 : cols;
    const float* xr = x + row * cols;
    float* orow = out + row * cols;
    float m = -INFINITY;
    for (uint64_t c = threadIdx.x; c < visible; c += 256) m = fmaxf(m, xr[c]);
    m = block_max(m, scratch);
    float sum = 0.f;
    for (uint64_t c = threadIdx.x; c < visible; c += 256) sum += expf(xr[c] - m);
    sum = block_sum(sum, scratch);
    const float inv = 1.0f / sum;
    for (uint64_t c = threadIdx.x; c < cols; c += 256) orow[c] = c < visible ? expf(xr[c] - m) * inv : 0.f;
}

}  // namespace

hipError_t launch_rms_norm(const float* x, const float* w, float* out, uint64_t rows, uint64_t hidden,
                           float eps, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    const bool vec = hidden % 4 == 0 && aligned16(x) && aligned16(w) && aligned16(out);
    const uint64_t h4 = hidden / 4;
    if (vec && rows <= 0x7fffffffu) {
        const auto args = [&](auto kernel) {
            kernel<<<static_cast<unsigned>(rows), 256, 0, s>>>(
                reinterpret_cast<const float4*>(x), reinterpret_cast<const float4*>(w),
                reinterpret_cast<float4*>(out), static_cast<uint32_t>(h4), static_cast<float>(hidden), eps);
        };
        if (h4 <= 256) { args(rms_norm_vec<1>); return hipGetLastError(); }
        if (h4 <= 512) { args(rms_norm_vec<2>); return hipGetLastError(); }
        if (h4 <= 1024) { args(rms_norm_vec<4>); return hipGetLastError(); }
        if (h4 <= 2048) { args(rms_norm_vec<8>); return hipGetLastError(); }
    }
    rms_norm_any<<<static_cast<unsigned>(rows), 256, 0, s>>>(x, w, out, hidden, eps);
    return hipGetLastError();
}

hipError_t launch_softmax(const float* x, float* out, uint64_t rows, uint64_t cols, bool causal,
                          uint64_t seq, uint64_t past_len, const uint32_t* dyn, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    const unsigned g = static_cast<unsigned>(rows);
    const uint32_t c = static_cast<uint32_t>(cols), q = static_cast<uint32_t>(seq),
                   p = static_cast<uint32_t>(past_len);
    if (cols <= 256 * 16) {
#define SL_SOFTMAX(V)                                                              \
    do {                                                                           \
        if (causal) softmax_regs<V, true><<<g, 256, 0, s>>>(x, out, c, q, p, dyn); \
        else softmax_regs<V, false><<<g, 256, 0, s>>>(x, out, c, q, p, dyn);       \
        return hipGetLastError();                                                  \
    } while (0)
        if (cols <= 256) SL_SOFTMAX(1);
        if (cols <= 512) SL_SOFTMAX(2);
        if (cols <= 1024) SL_SOFTMAX(4);
        if (cols <= 2048) SL_SOFTMAX(8);
        SL_SOFTMAX(16);
#undef SL_SOFTMAX
    }
    if (causal) softmax_any<true><<<g, 256, 0, s>>>(x, out, cols, seq, past_len, dyn);
    else softmax_any<false><<<g, 256, 0, s>>>(x, out, cols, seq, past_len, dyn);
    return hipGetLastError();
}

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_norm_softmax() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&rms_norm_any));
}

}  // namespace slhip
