// Prefill projections Y[batch, rows] = X[batch, cols] . A^T (batch >= 5) on
// gfx950, fp32 / BF16 / int8-per-row weights, fp32 accumulation.
//
// fp32 weights (the prefill of every config): FP32 MFMA
// (v_mfma_f32_32x32x2_f32). A 128 (tokens) x 128 (rows) output tile per
// 256-thread block, 2 x 2 waves of 64 x 64 (2 x 2 MFMA tiles each); K in
// steps of 16 through LDS, k-major ([k][m], [k][n]) so each MFMA operand is
// one conflict-free ds_read_b32 per lane; the next K step's global loads are
// in flight (registers) while the current one is multiplied.
// fp32 weights with at most 16 rows: gemm_skinny_kernel (lanes over columns).
// Fewer 128 x 128 tiles than CUs: K split into chunks (partials + an ordered
// sum). The prefill GLU: gate and up in one MFMA kernel with silu(g) * u in
// the epilogue.
// BF16 / int8 weights: the LDS-tiled FMA kernel below (64 x 64 tile, 4 x 4
// outputs per thread). int8 rows are scaled after the sum (scale * sum(q x),
// as the reference's qr_gemm_i8, native/rocm/bridge.cpp:620-653).
#include "common.h"

namespace qr {
namespace {

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));

// LDS rows of 132 floats: the two lane halves of an MFMA operand read take
// rows k and k + 8 (8 * 132 = 32 banks apart), and the four k-quads a wave
// stores land 16 banks apart, so neither side has bank conflicts.
constexpr int MM = 128, MN = 128, MK = 16, MPAD = 4;

// One 16-deep K step of two 64-row blocks into registers: thread t loads row
// t / 4 of each (v[0] from `top`, v[1] from `bottom`), 4 consecutive k at
// (t % 4) * 4; zero outside the matrix or past k_end.
__device__ __forceinline__ void mfma_load(const float* top, int top_r0, const float* bottom, int bottom_r0, int rows,
                                          int cols, int k0, int k_end, f4v (&v)[2]) {
    const int t = threadIdx.x, kq = (t & 3) * 4, k = k0 + kq;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float* m = i ? bottom : top;
        const int r = (i ? bottom_r0 : top_r0) + (t >> 2);
        if (r < rows && k + 3 < k_end) {
            v[i] = *reinterpret_cast<const f4v*>(m + size_t(r) * cols + k);
        } else {
            f4v z = {0.f, 0.f, 0.f, 0.f};
            for (int e = 0; e < 4; ++e)
                if (r < rows && k + e < k_end) z[e] = m[size_t(r) * cols + k + e];
            v[i] = z;
        }
    }
}
__device__ __forceinline__ void mfma_store(float (*lds)[MM + MPAD], const f4v (&v)[2]) {
    const int t = threadIdx.x, kq = (t & 3) * 4;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = (t >> 2) + 64 * i;
#pragma unroll
        for (int e = 0; e < 4; ++e) lds[kq + e][r] = v[i][e];
    }
}

// GLU = false: Y = X A^T, a 128 x 128 tile per block (the wave's 64 x 64
// sub-tile is 2 x 2 MFMA tiles). GLU = true: product = silu(X G^T) * (X U^T)
// for 128 tokens x 64 rows, the weight tile being [64 gate rows | the same 64
// up rows]: the wave's sub-tile is 64 tokens x 32 rows of gate (j = 0) and of
// up (j = 1), so a gate value and its up partner sit in the same register of
// the same lane. blockIdx.z: the K split [z * kchunk, +kchunk); with more than
// one split the block writes its partial sums to y + z * batch * rows.
template <bool GLU>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(float* y, const float* a, const float* a2, const float* x,
                                                        int rows, int cols, int batch, int kchunk) {
    __shared__ float xs[2][MK][MM + MPAD];
    __shared__ float ws[2][MK][MN + MPAD];
    constexpr int NT = GLU ? 64 : MN;  // output rows per block
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * (GLU ? 32 : 64);
    const int m0 = blockIdx.y * MM, n0 = blockIdx.x * NT;
    const int kbeg = int(blockIdx.z) * kchunk, kend = min(cols, kbeg + kchunk);
    float* out = y + size_t(blockIdx.z) * size_t(batch) * size_t(rows);
    const float* wbot = GLU ? a2 : a;
    const int wbot_r0 = GLU ? n0 : n0 + 64;
    f16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    f4v xv[2], wv[2];
    mfma_load(x, m0, x, m0 + 64, batch, cols, kbeg, kend, xv);
    mfma_load(a, n0, wbot, wbot_r0, rows, cols, kbeg, kend, wv);
    mfma_store(xs[0], xv);
    mfma_store(ws[0], wv);
    __syncthreads();
    int buf = 0;
    for (int k0 = kbeg; k0 < kend; k0 += MK) {
        const bool more = k0 + MK < kend;
        if (more) {  // next K step in flight while this one is multiplied
            mfma_load(x, m0, x, m0 + 64, batch, cols, k0 + MK, kend, xv);
            mfma_load(a, n0, wbot, wbot_r0, rows, cols, k0 + MK, kend, wv);
        }
#pragma unroll
        for (int kk = 0; kk < MK / 2; ++kk) {
            const int k = kk + (MK / 2) * (lane >> 5);  // A[i = lane % 32][k], B[k][j = lane % 32]
            float av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) av[i] = xs[buf][k][wm + 32 * i + (lane & 31)];
#pragma unroll
            for (int j = 0; j < 2; ++j) bv[j] = ws[buf][k][(GLU ? 64 * j + wn : wn + 32 * j) + (lane & 31)];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            mfma_store(xs[buf ^ 1], xv);
            mfma_store(ws[buf ^ 1], wv);
        }
        __syncthreads();
        buf ^= 1;
    }
    // D[i][j]: lane l, register r holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < (GLU ? 1 : 2); ++j) {
            const int n = n0 + wn + 32 * j + (lane & 31);
            if (n >= rows) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < batch) out[size_t(m) * rows + n] = GLU ? siluf_(acc[i][0][r]) * acc[i][1][r] : acc[i][j][r];
            }
        }
}

// y = the sum of `splits` partial results (in split order), float4 at a time.
__global__ __launch_bounds__(256) void split_sum_kernel(float* y, const float* parts, int splits, size_t n4) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n4) return;
    const f4v* p = reinterpret_cast<const f4v*>(parts);
    f4v s = p[i];
    for (int k = 1; k < splits; ++k) s += p[size_t(k) * n4 + i];
    reinterpret_cast<f4v*>(y)[i] = s;
}

// K splits of an fp32 MFMA GEMM: fewer 128 x 128 tiles than CUs leave CUs
// idle, so K is cut into up to 4 chunks (multiples of the 16-deep step) until
// there are about two blocks per CU.
int mfma_splits(int rows, int cols, int batch, int& kchunk) {
    const long tiles = long(ceil_div(rows, MN)) * long(ceil_div(batch, MM));
    int splits = 1;
    if (rows % 4 == 0)
        while (splits < 4 && tiles * splits < 2 * 256 && cols / (splits + 1) >= 4 * MK) ++splits;
    kchunk = int(ceil_div(ceil_div(cols, splits), MK)) * MK;
    return int(ceil_div(cols, kchunk));
}

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

// fp32 weights with few rows (<= 16: the DeltaNet a / b projections) over many
// tokens: a 128-row MFMA tile would be mostly empty, so each wave takes 4
// tokens, its lanes stride the columns with coalesced float4 loads of x and
// of every weight row, and the 4 x 16 per-lane partial dots are summed over
// the 64 lanes through LDS (one (token, row) output per lane).
constexpr int SK_ROWS = 16, SK_TOK = 4;
__global__ __launch_bounds__(256) void gemm_skinny_kernel(float* y, const float* a, const float* x, int rows, int cols,
                                                          int batch) {
    __shared__ float part[4][64][SK_ROWS * SK_TOK + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = (int(blockIdx.x) * 4 + wave) * SK_TOK;
    float acc[SK_TOK][SK_ROWS] = {};
    for (int c = lane * 4; c < cols; c += 256) {
        f4v xv[SK_TOK];
#pragma unroll
        for (int t = 0; t < SK_TOK; ++t)
            xv[t] = m0 + t < batch ? *reinterpret_cast<const f4v*>(x + size_t(m0 + t) * cols + c) : f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < SK_ROWS; ++r) {
            if (r >= rows) break;
            const f4v av = *reinterpret_cast<const f4v*>(a + size_t(r) * cols + c);
#pragma unroll
            for (int t = 0; t < SK_TOK; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[t][r] = fmaf(xv[t][e], av[e], acc[t][r]);
        }
    }
#pragma unroll
    for (int t = 0; t < SK_TOK; ++t)
#pragma unroll
        for (int r = 0; r < SK_ROWS; ++r) part[wave][lane][t * SK_ROWS + r] = acc[t][r];
    __syncthreads();
    const int t = lane / SK_ROWS, r = lane % SK_ROWS;
    float sum = 0.f;
    for (int j = 0; j < 64; ++j) sum += part[wave][j][lane];
    if (m0 + t < batch && r < rows) y[size_t(m0 + t) * rows + r] = sum;
}

}  // namespace

bool gemm_preferred(WeightType, int, int, int batch) { return batch > 4; }

static bool mfma_ok(const void* a, const float* x, int cols) {
    return cols % 4 == 0 && (reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(x)) % 16 == 0;
}

size_t gemm_scratch(WeightType t, int rows, int cols, int batch) {
    if (t != WeightType::F32 || rows <= SK_ROWS) return 0;
    int kchunk;
    const int splits = mfma_splits(rows, cols, batch, kchunk);
    return splits > 1 ? size_t(splits) * size_t(rows) * size_t(batch) : 0;
}

int gemm(hipStream_t s, WeightType t, float* y, const void* a, const float* x, int rows, int cols, int batch,
         float* work, size_t work_len) {
    dim3 grid(ceil_div(rows, BN), ceil_div(batch, BM));
    switch (t) {
    case WeightType::F32:
        // 16-byte aligned rows for the vector loads
        if (mfma_ok(a, x, cols)) {
            const float* af = static_cast<const float*>(a);
            if (rows <= SK_ROWS) {
                hipLaunchKernelGGL(gemm_skinny_kernel, dim3(ceil_div(batch, 4 * SK_TOK)), dim3(256), 0, s, y, af, x,
                                   rows, cols, batch);
                break;
            }
            int kchunk;
            const int splits = mfma_splits(rows, cols, batch, kchunk);
            const dim3 g(ceil_div(rows, MN), ceil_div(batch, MM), unsigned(splits));
            if (splits == 1) {
                hipLaunchKernelGGL(gemm_mfma_kernel<false>, g, dim3(256), 0, s, y, af, af, x, rows, cols, batch, kchunk);
                break;
            }
            const size_t n = size_t(rows) * size_t(batch);
            if (!work || work_len < size_t(splits) * n) return int(hipErrorInvalidValue);
            hipLaunchKernelGGL(gemm_mfma_kernel<false>, g, dim3(256), 0, s, work, af, af, x, rows, cols, batch, kchunk);
            if (hipError_t e = hipGetLastError()) return int(e);
            hipLaunchKernelGGL(split_sum_kernel, dim3(ceil_div(long(n / 4), 256)), dim3(256), 0, s, y,
                               static_cast<const float*>(work), splits, n / 4);
            break;
        }
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

bool gemm_glu_fused(WeightType t, const void* gate, const void* up, const float* x, int rows, int cols, int batch) {
    return t == WeightType::F32 && gemm_preferred(t, rows, cols, batch) && mfma_ok(gate, x, cols) &&
           mfma_ok(up, x, cols);
}

int gemm_glu(hipStream_t s, float* product, const float* gate, const float* up, const float* x, int rows, int cols,
             int batch) {
    const dim3 g(ceil_div(rows, 64), ceil_div(batch, MM), 1);
    hipLaunchKernelGGL(gemm_mfma_kernel<true>, g, dim3(256), 0, s, product, gate, up, x, rows, cols, batch, cols);
    return int(hipGetLastError());
}

}  // namespace qr
