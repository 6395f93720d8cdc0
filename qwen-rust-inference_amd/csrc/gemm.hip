// Prefill projections Y[batch, rows] = X[batch, cols] . A^T (batch >= 5) on
// gfx950, fp32 / BF16 / int8-per-row weights, fp32 accumulation.
//
// LDS-tiled kernel: a 64 (tokens) x 64 (rows) output tile per 256-thread
// block, K in steps of 16 staged transposed in LDS, 4 x 4 outputs per thread.
// int8 rows are scaled after the sum (scale * sum(q x), as the reference's
// qr_gemm_i8, native/rocm/bridge.cpp:620-653).
#include "common.h"

namespace qr {
namespace {

constexpr int BM = 64, BN = 64, BK = 16;

template <WeightType T>
__device__ __forceinline__ float weight_at(const void* a, int rows, int cols, long r, long k) {
    if constexpr (T == WeightType::F32) return reinterpret_cast<const float*>(a)[size_t(r) * cols + k];
    if constexpr (T == WeightType::BF16)
        return __uint_as_float(uint32_t(reinterpret_cast<const uint16_t*>(a)[size_t(r) * cols + k]) << 16);
    return float(reinterpret_cast<const int8_t*>(reinterpret_cast<const float*>(a) + rows)[size_t(r) * cols + k]);
}

template <WeightType T>
__global__ __launch_bounds__(256) void gemm_tiled_kernel(float* y, const void* a, const float* x, int rows, int cols,
                                                         int batch) {
    __shared__ float xs[BK][BM + 4];
    __shared__ float as[BK][BN + 4];
    const int tid = threadIdx.x;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int ty = tid / 16, tx = tid % 16;
    float acc[4][4] = {};
    const int lm = tid / 4, lk = (tid % 4) * 4;
    for (int k0 = 0; k0 < cols; k0 += BK) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int k = k0 + lk + e;
            const int m = m0 + lm, n = n0 + lm;
            xs[lk + e][lm] = (m < batch && k < cols) ? x[size_t(m) * cols + k] : 0.f;
            as[lk + e][lm] = (n < rows && k < cols) ? weight_at<T>(a, rows, cols, n, k) : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < BK; ++k) {
            float xv[4], av[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xv[i] = xs[k][ty * 4 + i];
                av[i] = as[k][tx * 4 + i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(xv[i], av[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty * 4 + i;
        if (m >= batch) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n >= rows) continue;
            float v = acc[i][j];
            if constexpr (T == WeightType::I8) v *= reinterpret_cast<const float*>(a)[n];
            y[size_t(m) * rows + n] = v;
        }
    }
}

}  // namespace

bool gemm_preferred(WeightType, int, int, int batch) { return batch > 4; }

int gemm(hipStream_t s, WeightType t, float* y, const void* a, const float* x, int rows, int cols, int batch) {
    dim3 grid(ceil_div(rows, BN), ceil_div(batch, BM));
    switch (t) {
    case WeightType::F32:
        hipLaunchKernelGGL(gemm_tiled_kernel<WeightType::F32>, grid, dim3(256), 0, s, y, a, x, rows, cols, batch);
        break;
    case WeightType::BF16:
        hipLaunchKernelGGL(gemm_tiled_kernel<WeightType::BF16>, grid, dim3(256), 0, s, y, a, x, rows, cols, batch);
        break;
    case WeightType::I8:
        hipLaunchKernelGGL(gemm_tiled_kernel<WeightType::I8>, grid, dim3(256), 0, s, y, a, x, rows, cols, batch);
        break;
    }
    return int(hipGetLastError());
}

}  // namespace qr
