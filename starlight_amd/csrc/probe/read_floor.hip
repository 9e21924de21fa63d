// Read floors: how long the plainest full-chip read of a given number of
// bytes takes on this GPU when it is one launch of a replayed HIP graph,
// the way every decode kernel runs. A kernel that must read B bytes in one
// launch cannot beat the floor for B, so the floor — not the 8 TB/s peak
// alone — shows how much of a latency-bound launch's time is its own.
//
// libstarlight_probe.so is a measurement library for bench.py, separate
// from libstarlight_hip.so: the device path never calls it.
//
// read_k: block b reads the 16-byte words [b * per, (b + 1) * per) of the
// range, 4 independent loads per thread per round, and folds them into one
// word that is stored only if it equals a value no test data holds (so the
// loads cannot be removed). Blocks of 512 threads, one per 64 KiB of the
// range, at least 256 and at most 2048 (every CU busy, about 8 KiB per
// thread at most in flight).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ __launch_bounds__(512) void read_k(const uint4* __restrict__ base, uint64_t n, uint64_t per,
                                             uint32_t* sink) {
    const uint64_t lo = static_cast<uint64_t>(blockIdx.x) * per;
    if (lo >= n) return;
    const uint64_t hi = lo + per < n ? lo + per : n;
    uint32_t acc = 0;
    for (uint64_t i = lo + threadIdx.x; i < hi; i += static_cast<uint64_t>(blockDim.x) * 4) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * blockDim.x;
            v[u] = j < hi ? base[j] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

constexpr uint32_t kMaxBlocks = 2048;

hipError_t launch_read(const void* p, uint64_t bytes, uint32_t* sink, hipStream_t s) {
    const uint64_t n = bytes / 16;
    uint64_t blocks = bytes / 65536;
    if (blocks < 256) blocks = 256;
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    const uint64_t per = (n + blocks - 1) / blocks;
    read_k<<<static_cast<unsigned>(blocks), 512, 0, s>>>(static_cast<const uint4*>(p), n, per, sink);
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
