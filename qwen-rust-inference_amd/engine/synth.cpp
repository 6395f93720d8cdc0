// Synthetic weights for the benchmark configs: a counter-based N(0, std)
// generator. Element i of (seed, stream) is a pure function of those three
// numbers (splitmix64 of a per-stream key plus the pair index, Box-Muller in
// double), so the values do not depend on how many threads fill the array.
#include <cmath>
#include <cstdint>
#include <thread>
#include <vector>

#include "../../include/qwen_engine.h"

namespace {
uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}
void fill(float* dst, uint64_t begin, uint64_t end, uint64_t key, float std_dev) {
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t i = begin & ~uint64_t(1); i < end; i += 2) {
        const uint64_t z = splitmix64(key + (i >> 1) * 0x9e3779b97f4a7c15ull);
        const double u1 = (double(z >> 40) + 0.5) / 16777216.0;
        const double u2 = (double(z & 0xffffffull) + 0.5) / 16777216.0;
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double v0 = r * std::cos(two_pi * u2), v1 = r * std::sin(two_pi * u2);
        if (i >= begin) dst[i] = float(v0 * std_dev);
        if (i + 1 >= begin && i + 1 < end) dst[i + 1] = float(v1 * std_dev);
    }
}
}  // namespace

extern "C" void qw_synth_normal(float* dst, uint64_t n, uint64_t seed, uint64_t stream, float std_dev, int threads) {
    const uint64_t key = splitmix64(seed * 0x632be59bd9b4e019ull ^ splitmix64(stream + 0x1234567ull));
    unsigned hw = std::thread::hardware_concurrency();
    int t = threads > 0 ? threads : int(hw ? hw : 1);
    if (n < (uint64_t(1) << 20) || t == 1) {
        fill(dst, 0, n, key, std_dev);
        return;
    }
    std::vector<std::thread> pool;
    const uint64_t per = ((n + uint64_t(t) - 1) / uint64_t(t) + 1) & ~uint64_t(1);
    for (int k = 0; k < t; ++k) {
        uint64_t b = uint64_t(k) * per, e = b + per < n ? b + per : n;
        if (b >= n) break;
        pool.emplace_back(fill, dst, b, e, key, std_dev);
    }
    for (auto& th : pool) th.join();
}
