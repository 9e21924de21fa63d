// Read floors: how long the plainest full-chip read of a given number of
// bytes takes on this GPU when it is one launch of a replayed HIP graph,
// the way every decode kernel runs. A kernel that must read B bytes in one
// launch cannot beat the floor for B, so the floor — not the 8 TB/s peak
// alone — shows how much of a latency-bound launch's time is its own.
//
// libstarlight_probe.so is a measurement library for bench.py, separate
// from libstarlight_hip.so: the device path never calls it.
//
// read_k: each thread issues its two 16-byte loads at once (block b of 512
// threads reads the 16 KiB at b * 16 KiB) and folds them into one word
// that is stored only if it equals a value no test data holds (so the loads
// cannot be removed). Of the plain reads measured on the MI355X (rounds of
// four loads per thread, 2 / 4 / 8 loads per thread all at once, and
// gfx950's global -> LDS loads), this form was the fastest or within 2% of
// it at every size from 4 to 134 MB.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr uint32_t kThreads = 512, kLoads = 2;

__global__ __launch_bounds__(512) void read_k(const uint4* __restrict__ base, uint64_t n, uint32_t* sink) {
    const uint64_t lo = static_cast<uint64_t>(blockIdx.x) * (kThreads * kLoads) + threadIdx.x;
    uint4 v[kLoads];
#pragma unroll
    for (uint32_t u = 0; u < kLoads; ++u) {
        const uint64_t j = lo + u * kThreads;
        v[u] = base[j < n ? j : n - 1];
    }
    uint32_t acc = 0;
#pragma unroll
    for (uint32_t u = 0; u < kLoads; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x9E3779B9u) sink[blockIdx.x % 2048] = acc;
}

hipError_t launch_read(const void* p, uint64_t bytes, uint32_t* sink, hipStream_t s) {
    const uint64_t n = bytes / 16;
    const uint64_t blocks = (n + kThreads * kLoads - 1) / (kThreads * kLoads);
    read_k<<<static_cast<unsigned>(blocks), kThreads, 0, s>>>(static_cast<const uint4*>(p), n, sink);
    return hipGetLastError();
}

// Captures `count` reads (ptrs[i], bytes[i]) as one graph, replays it once
// to warm up, then `trials` times, and returns the best replay's time in
// microseconds.
int time_reads(const void* const* ptrs, const uint64_t* bytes, uint32_t count, uint32_t* sink, hipStream_t s,
               uint32_t trials, float* us) {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    for (uint32_t i = 0; e == hipSuccess && i < count; ++i) e = launch_read(ptrs[i], bytes[i], sink, s);
    const hipError_t end = hipStreamEndCapture(s, &graph);
    if (e == hipSuccess) e = end;
    if (e == hipSuccess) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipGraphLaunch(exec, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    float best = 1e30f;
    for (uint32_t t = 0; e == hipSuccess && t < trials; ++t) {
        e = hipEventRecord(e0, s);
        if (e == hipSuccess) e = hipGraphLaunch(exec, s);
        if (e == hipSuccess) e = hipEventRecord(e1, s);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e == hipSuccess && ms < best) best = ms;
    }
    if (e1) (void)hipEventDestroy(e1);
    if (e0) (void)hipEventDestroy(e0);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return static_cast<int>(e);
    *us = best * 1000.0f;
    return 0;
}

}  // namespace

extern "C" {

// Reads `bytes` at base, base + stride, ... (copies regions, rotated) as
// `launches` launches of one graph; *us_per_launch = best replay / launches.
// With copies * stride beyond the 256 MB MALL every launch reads from HBM.
// `sink` is a device buffer of at least 2048 words. Returns a hipError_t.
int slp_read_floor(const void* base, uint64_t bytes, uint64_t stride, uint32_t copies, uint32_t launches,
                   uint32_t* sink, void* stream, float* us_per_launch) {
    if (base == nullptr || bytes < 16 || copies == 0 || launches == 0 || launches > 4096 || us_per_launch == nullptr ||
        reinterpret_cast<uintptr_t>(base) % 16 != 0 || stride % 16 != 0)
        return static_cast<int>(hipErrorInvalidValue);
    const void* ptrs[4096];
    uint64_t sizes[4096];
    for (uint32_t i = 0; i < launches; ++i) {
        ptrs[i] = static_cast<const uint8_t*>(base) + static_cast<uint64_t>(i % copies) * stride;
        sizes[i] = bytes;
    }
    float us = 0.f;
    const int rc = time_reads(ptrs, sizes, launches, sink, static_cast<hipStream_t>(stream), 5, &us);
    if (rc == 0) *us_per_launch = us / static_cast<float>(launches);
    return rc;
}

// One graph of `count` reads, read i of bytes[i] at ptrs[i], in order;
// *us_total = the best replay. Returns a hipError_t.
int slp_read_sequence(const void* const* ptrs, const uint64_t* bytes, uint32_t count, uint32_t* sink,
                      void* stream, float* us_total) {
    if (ptrs == nullptr || bytes == nullptr || count == 0 || us_total == nullptr)
        return static_cast<int>(hipErrorInvalidValue);
    for (uint32_t i = 0; i < count; ++i)
        if (ptrs[i] == nullptr || bytes[i] < 16 || reinterpret_cast<uintptr_t>(ptrs[i]) % 16 != 0)
            return static_cast<int>(hipErrorInvalidValue);
    return time_reads(ptrs, bytes, count, sink, static_cast<hipStream_t>(stream), 5, us_total);
}

}  // extern "C"
