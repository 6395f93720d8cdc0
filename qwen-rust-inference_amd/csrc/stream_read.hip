// Attainable HBM read bandwidth on this GPU: a stream-read kernel in the
// decode kernel's load pattern (16-byte non-temporal buffer loads, 16 in
// flight per lane, each wave streaming a contiguous slice), over a buffer far
// larger than the L2s and the memory-side cache. Prints one JSON line.
// Usage: stream_read [MiB (multiple of 1024)] [repetitions]
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <vector>

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t Rs;
__device__ f4 buffer_load_f4(Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.load.v4f32");

namespace {
constexpr int kNT = 2, BLOCKS = 2048, THREADS = 256, WAVES = BLOCKS * THREADS / 64, STEP = 16 * 1024;

// one 1 GiB chunk: WAVES slices of `slice` bytes (a multiple of STEP)
__global__ __launch_bounds__(THREADS) void read_chunk(const float* p, unsigned slice, float* sink) {
    const Rs r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, -1, 0x00020000);
    const unsigned wave = blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned base = wave * slice;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    for (unsigned o = 0; o < slice; o += STEP) {
        f4 v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = buffer_load_f4(r, base + o + 1024u * unsigned(k) + 16u * lane, 0, kNT);
#pragma unroll
        for (int k = 0; k < 16; ++k) acc += v[k];
    }
    if (acc.x + acc.y + acc.z + acc.w == 1234.5f) sink[blockIdx.x] = 1.f;  // keeps the loads
}

int check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "stream_read: %s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
    return 0;
}
}  // namespace

int main(int argc, char** argv) {
    const size_t mib = argc > 1 ? size_t(atoll(argv[1])) : 4096;
    const int reps = argc > 2 ? atoi(argv[2]) : 10;
    const size_t chunk = size_t(1) << 30;
    if (mib == 0 || (mib << 20) % chunk || reps < 1) {
        fprintf(stderr, "stream_read: size must be a positive multiple of 1024 MiB, reps >= 1\n");
        return 2;
    }
    const size_t bytes = mib << 20;
    float *buf = nullptr, *sink = nullptr;
    check(hipMalloc(&buf, bytes), "hipMalloc");
    check(hipMalloc(&sink, BLOCKS * sizeof(float)), "hipMalloc");
    check(hipMemset(buf, 0, bytes), "hipMemset");
    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "event");
    check(hipEventCreate(&e1), "event");
    const unsigned slice = unsigned(chunk / WAVES);
    static_assert((size_t(1) << 30) / WAVES % STEP == 0, "slices of whole steps");
    std::vector<float> us;
    for (int rep = 0; rep <= reps; ++rep) {
        check(hipEventRecord(e0, nullptr), "record");
        for (size_t o = 0; o < bytes; o += chunk)
            read_chunk<<<BLOCKS, THREADS>>>(buf + o / sizeof(float), slice, sink);
        check(hipGetLastError(), "launch");
        check(hipEventRecord(e1, nullptr), "record");
        check(hipEventSynchronize(e1), "sync");
        float ms = 0.f;
        check(hipEventElapsedTime(&ms, e0, e1), "elapsed");
        if (rep) us.push_back(ms * 1e3f);  // the first pass warms up
    }
    std::sort(us.begin(), us.end());
    const float med = us[us.size() / 2];
    printf("{\"bytes\": %zu, \"reps\": %d, \"median_us\": %.1f, \"gbs\": %.1f}\n", bytes, reps, med,
           double(bytes) / (double(med) * 1e3));
    check(hipFree(buf), "free");
    check(hipFree(sink), "free");
    return 0;
}
