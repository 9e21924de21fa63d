// Elementwise kernels: Add, Mul, Scale, Silu (reference/elementwise.rs:10-74)
// and the fused silu(g)*u epilogue used by SwiGlu.
//
// Each kernel streams 16-byte vectors when every pointer is 16-byte aligned
// (grid-stride over float4, scalar tail); otherwise it runs the scalar form.
// Arithmetic is the reference's, one IEEE op per step and no contraction
// (built with -ffp-contract=off), so Add/Mul/Scale are bit-identical to it and
// Silu differs only by the device expf.
#include "common.h"
#include "kernels.h"

namespace slhip {
namespace {

enum class Ew { Add, Mul, Scale, Silu, SiluMul, Zero, Copy };

template <Ew OP>
__device__ __forceinline__ float apply(float a, float b, float factor) {
    if constexpr (OP == Ew::Add) return a + b;
    if constexpr (OP == Ew::Mul) return a * b;
    if constexpr (OP == Ew::Scale) return a * factor;
    // silu_scalar (elementwise.rs:10-12): x * (1 / (1 + exp(-x)))
    if constexpr (OP == Ew::Silu) return a * (1.0f / (1.0f + expf(-a)));
    if constexpr (OP == Ew::SiluMul) return (a * (1.0f / (1.0f + expf(-a)))) * b;
    if constexpr (OP == Ew::Copy) return a;
    return 0.0f;
}

template <Ew OP>
__global__ __launch_bounds__(256) void ew_vec4(const float4* __restrict__ a, const float4* __restrict__ b,
                                               float4* __restrict__ out, uint64_t n4, float factor) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 x = OP == Ew::Zero ? make_float4(0.f, 0.f, 0.f, 0.f) : a[i];
        float4 y = (OP == Ew::Add || OP == Ew::Mul || OP == Ew::SiluMul) ? b[i] : x;
        float4 r;
        r.x = apply<OP>(x.x, y.x, factor);
        r.y = apply<OP>(x.y, y.y, factor);
        r.z = apply<OP>(x.z, y.z, factor);
        r.w = apply<OP>(x.w, y.w, factor);
        stream_store(out + i, r);
    }
}

template <Ew OP>
__global__ __launch_bounds__(256) void ew_scalar(const float* __restrict__ a, const float* __restrict__ b,
                                                 float* __restrict__ out, uint64_t begin, uint64_t n,
                                                 float factor) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = begin + static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        float x = OP == Ew::Zero ? 0.f : a[i];
        float y = (OP == Ew::Add || OP == Ew::Mul || OP == Ew::SiluMul) ? b[i] : x;
        out[i] = apply<OP>(x, y, factor);
    }
}

// The scalar form: 256 CUs x 8 resident blocks of 256 threads keeps every CU
// busy; larger tensors loop inside the kernel. The vector form gives each
// thread one float4 up to 2^28 of them (a 4096 x 14336 Add: 118 us, 5.95
// TB/s on MI355X, against 125 us with the grid capped at 2048 blocks and
// each thread looping); the loop covers anything larger.
constexpr unsigned kGridCap = 256 * 8;
constexpr unsigned kVecGridCap = 1u << 20;

template <Ew OP>
hipError_t launch_ew(const float* a, const float* b, float* out, uint64_t n, float factor, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const bool vec = aligned16(out) && (a == nullptr || aligned16(a)) && (b == nullptr || aligned16(b));
    uint64_t done = 0;
    if (vec && n >= 4) {
        const uint64_t n4 = n / 4;
        ew_vec4<OP><<<grid_for(n4, 256, kVecGridCap), 256, 0, s>>>(
            reinterpret_cast<const float4*>(a), reinterpret_cast<const float4*>(b),
            reinterpret_cast<float4*>(out), n4, factor);
        done = n4 * 4;
    }
    if (done < n)
        ew_scalar<OP><<<grid_for(n - done, 256, kGridCap), 256, 0, s>>>(a, b, out, done, n, factor);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_add(const float* a, const float* b, float* out, uint64_t n, hipStream_t s) {
    return launch_ew<Ew::Add>(a, b, out, n, 0.f, s);
}
hipError_t launch_mul(const float* a, const float* b, float* out, uint64_t n, hipStream_t s) {
    return launch_ew<Ew::Mul>(a, b, out, n, 0.f, s);
}
hipError_t launch_scale(const float* x, float* out, uint64_t n, float factor, hipStream_t s) {
    return launch_ew<Ew::Scale>(x, nullptr, out, n, factor, s);
}
hipError_t launch_silu(const float* x, float* out, uint64_t n, hipStream_t s) {
    return launch_ew<Ew::Silu>(x, nullptr, out, n, 0.f, s);
}
hipError_t launch_silu_mul(const float* g, const float* u, float* h, uint64_t n, hipStream_t s) {
    return launch_ew<Ew::SiluMul>(g, u, h, n, 0.f, s);
}
namespace {
constexpr uint32_t kSetWords = 240;
struct Words {
    uint32_t v[kSetWords];
};
// dst[i] = w.v[i], i < count: the values travel in the kernel arguments, so
// the host array may change as soon as the launch returns.
__global__ void set_words(uint32_t* __restrict__ dst, Words w, uint32_t count) {
    const uint32_t i = threadIdx.x;
    if (i < count) dst[i] = w.v[i];
}
}  // namespace

hipError_t launch_set_words(uint32_t* dst, const uint32_t* values, uint64_t count, hipStream_t s) {
    for (uint64_t done = 0; done < count; done += kSetWords) {
        const uint32_t n = static_cast<uint32_t>(count - done < kSetWords ? count - done : kSetWords);
        Words w{};
        for (uint32_t i = 0; i < n; ++i) w.v[i] = values[done + i];
        set_words<<<1, 256, 0, s>>>(dst + done, w, n);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_fill_zero(float* out, uint64_t n, hipStream_t s) {
    return launch_ew<Ew::Zero>(nullptr, nullptr, out, n, 0.f, s);
}
hipError_t launch_copy(const float* src, float* dst, uint64_t n, hipStream_t s) {
    return launch_ew<Ew::Copy>(src, nullptr, dst, n, 0.f, s);
}

// Loads this file's code object now: HIP loads one at the first use of
// any of its kernels, which otherwise lands inside the first submission
// that needs it (about 1-2 ms each, more for large objects).
hipError_t load_code_elementwise() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&set_words));
}

}  // namespace slhip
