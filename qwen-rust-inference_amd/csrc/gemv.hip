// Decode projections (1..8 tokens) on gfx950: y[t, r] = sum_j A[r, j] x[t, j]
// for fp32, BF16 and int8-per-row weights, plus the grouped, GLU and
// add+RMSNorm-tail variants of the bridge ABI.
//
// Layout: one wavefront owns R consecutive rows. Each lane owns the 16-byte
// chunks lane, lane+64, ... of a row (4 fp32 / 8 BF16 / 16 int8 columns per
// chunk), so every load instruction of a wave reads 1 KiB of contiguous
// weights. All V*R chunks of a wave's rows are issued before the first FMA
// (V*R = 8 chunks = 8 KiB in flight per wave, one row from 8 chunks a lane), the partial dot products are
// reduced with a wave64 butterfly, and lane r writes row r. The weights are
// streamed once (nontemporal loads: they are not reused within a token); the
// input vector is re-read from L1/L2.
#include "common.h"

namespace qr {
namespace {

template <WeightType T>
struct Elem;
template <>
struct Elem<WeightType::F32> {
    static constexpr int E = 4;  // columns per 16-byte chunk
};
template <>
struct Elem<WeightType::BF16> {
    static constexpr int E = 8;
};
template <>
struct Elem<WeightType::I8> {
    static constexpr int E = 16;
};

__device__ __forceinline__ uint4 load_stream(const uint4* p) {
    uint4 v;
    v.x = __builtin_nontemporal_load(&p->x);
    v.y = __builtin_nontemporal_load(&p->y);
    v.z = __builtin_nontemporal_load(&p->z);
    v.w = __builtin_nontemporal_load(&p->w);
    return v;
}

// Widen one raw chunk to E floats.
template <WeightType T>
__device__ __forceinline__ void widen(const uint4& u, float* v);
template <>
__device__ __forceinline__ void widen<WeightType::F32>(const uint4& u, float* v) {
    v[0] = __uint_as_float(u.x);
    v[1] = __uint_as_float(u.y);
    v[2] = __uint_as_float(u.z);
    v[3] = __uint_as_float(u.w);
}
template <>
__device__ __forceinline__ void widen<WeightType::BF16>(const uint4& u, float* v) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
template <>
__device__ __forceinline__ void widen<WeightType::I8>(const uint4& u, float* v) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) v[4 * i + b] = float(int8_t((w[i] >> (8 * b)) & 0xff));
    }
}

// Row r's first weight byte and (int8) scale.
template <WeightType T>
__device__ __forceinline__ const char* row_ptr(const void* a, int rows, int cols, long r) {
    if constexpr (T == WeightType::F32) return reinterpret_cast<const char*>(a) + size_t(r) * size_t(cols) * 4;
    if constexpr (T == WeightType::BF16) return reinterpret_cast<const char*>(a) + size_t(r) * size_t(cols) * 2;
    return reinterpret_cast<const char*>(a) + size_t(rows) * 4 + size_t(r) * size_t(cols);
}
template <WeightType T>
__device__ __forceinline__ float row_scale(const void* a, long r) {
    if constexpr (T == WeightType::I8) return reinterpret_cast<const float*>(a)[r];
    return 1.f;
}

__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct GemvParams {
    const void* a[kGroupMax];
    float* y[kGroupMax];
    int rows[kGroupMax];
    int first[kGroupMax + 1];  // first row group (wave) of each item
    int count;
    const float* x;
    int cols;
    const void* up;  // GLU: a[0] = gate, up = up, y[0] = product
    QrAddNormPost post;
    unsigned* ticket;
};

enum Mode { kPlain = 0, kGlu = 1, kAddNorm = 2 };

// The add+RMSNorm tail, run by the last block to finish (reference
// native/rocm/reference.h:194-200 for the arithmetic): sum = u + v and
// norm = (sum * r) * (w + offset), r = 1 / sqrt(mean(sum^2) + eps).
__device__ void add_norm_tail(const GemvParams& p, int d) {
    __shared__ float red[16];
    __shared__ int last;
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        unsigned prev = atomicAdd(p.ticket, 1u);
        last = prev == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    const QrAddNormPost& q = p.post;
    float ss = 0.f;
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        float s = load_coherent(q.u + i) + load_coherent(q.v + i);
        q.sum[i] = s;
        ss += s * s;
    }
    ss = block_sum(ss, red);
    float r = 1.f / sqrtf(ss / float(d) + q.eps);
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        float s = load_coherent(q.u + i) + load_coherent(q.v + i);
        q.norm[i] = (s * r) * (q.weight[i] + q.offset);
    }
    if (threadIdx.x == 0) atomicExch(p.ticket, 0u);  // ready for the next launch
}

template <WeightType T, int V, int R, int NB, int MODE>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
    constexpr int E = Elem<T>::E;
    constexpr int M = MODE == kGlu ? 2 : 1;  // matrices read per row
    const int lane = threadIdx.x & 63;
    const int g = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int cols = p.cols, chunks = cols / E;
    if (g < p.first[p.count]) {
        int item = 0;
        while (item + 1 < p.count && g >= p.first[item + 1]) ++item;
        const int rows = p.rows[item];
        const long r0 = long(g - p.first[item]) * R;
        const void* mats[2] = {p.a[item], MODE == kGlu ? p.up : nullptr};
        // Issue every weight load of this wave first.
        uint4 w[M][R][V];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint4* row = reinterpret_cast<const uint4*>(row_ptr<T>(mats[m], rows, cols, r0 + r));
                const bool live = r0 + r < rows;
#pragma unroll
                for (int c = 0; c < V; ++c) {
                    const int chunk = lane + 64 * c;
                    w[m][r][c] = live && (V * 64 == chunks || chunk < chunks) ? load_stream(row + chunk)
                                                                              : make_uint4(0, 0, 0, 0);
                }
            }
        float acc[M][R][NB];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int t = 0; t < NB; ++t) acc[m][r][t] = 0.f;
#pragma unroll
        for (int c = 0; c < V; ++c) {
            const int chunk = lane + 64 * c;
            if (V * 64 != chunks && chunk >= chunks) break;
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                float xv[E];
                const float4* xp = reinterpret_cast<const float4*>(p.x + size_t(t) * cols + size_t(chunk) * E);
#pragma unroll
                for (int e = 0; e < E / 4; ++e) {
                    float4 q = xp[e];
                    xv[4 * e] = q.x;
                    xv[4 * e + 1] = q.y;
                    xv[4 * e + 2] = q.z;
                    xv[4 * e + 3] = q.w;
                }
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float wv[E];
                        widen<T>(w[m][r][c], wv);
                        float s = acc[m][r][t];
#pragma unroll
                        for (int e = 0; e < E; ++e) s = fmaf(wv[e], xv[e], s);
                        acc[m][r][t] = s;
                    }
            }
        }
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int t = 0; t < NB; ++t) acc[m][r][t] = wave_sum(acc[m][r][t]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const long row = r0 + r;
            if (lane < NB && row < rows) {
                const int t = lane;
                float v0 = 0.f, v1 = 0.f;
#pragma unroll
                for (int tt = 0; tt < NB; ++tt)
                    if (tt == t) {
                        v0 = acc[0][r][tt];
                        v1 = acc[M - 1][r][tt];
                    }
                if constexpr (MODE == kGlu) {
                    p.y[item][size_t(t) * rows + row] =
                        siluf_(row_scale<T>(mats[0], row) * v0) * (row_scale<T>(mats[1], row) * v1);
                } else {
                    p.y[item][size_t(t) * rows + row] = row_scale<T>(mats[0], row) * v0;
                }
            }
        }
    }
    if constexpr (MODE == kAddNorm) add_norm_tail(p, p.rows[0]);
}

// Generic fallback for shapes the chunked kernel does not take (columns not a
// multiple of the chunk, unaligned buffers, very long rows): one block per
// (row, token), columns strided over the block.
template <WeightType T, int MODE>
__global__ __launch_bounds__(256) void gemv_generic(GemvParams p) {
    __shared__ float red[16];
    const int rows = p.rows[0], cols = p.cols;
    const long row = blockIdx.x;
    const int t = blockIdx.y;
    const float* x = p.x + size_t(t) * cols;
    float s0 = 0.f, s1 = 0.f;
    for (int j = threadIdx.x; j < cols; j += blockDim.x) {
        float w0, w1 = 0.f;
        if constexpr (T == WeightType::F32) {
            w0 = reinterpret_cast<const float*>(p.a[0])[size_t(row) * cols + j];
            if (MODE == kGlu) w1 = reinterpret_cast<const float*>(p.up)[size_t(row) * cols + j];
        } else if constexpr (T == WeightType::BF16) {
            w0 = __uint_as_float(uint32_t(reinterpret_cast<const uint16_t*>(p.a[0])[size_t(row) * cols + j]) << 16);
            if (MODE == kGlu)
                w1 = __uint_as_float(uint32_t(reinterpret_cast<const uint16_t*>(p.up)[size_t(row) * cols + j]) << 16);
        } else {
            w0 = float(reinterpret_cast<const int8_t*>(row_ptr<T>(p.a[0], rows, cols, row))[j]);
            if (MODE == kGlu) w1 = float(reinterpret_cast<const int8_t*>(row_ptr<T>(p.up, rows, cols, row))[j]);
        }
        s0 = fmaf(w0, x[j], s0);
        s1 = fmaf(w1, x[j], s1);
    }
    s0 = block_sum(s0, red);
    s1 = block_sum(s1, red);
    if (threadIdx.x == 0) {
        if constexpr (MODE == kGlu)
            p.y[0][size_t(t) * rows + row] = siluf_(row_scale<T>(p.a[0], row) * s0) * (row_scale<T>(p.up, row) * s1);
        else
            p.y[0][size_t(t) * rows + row] = row_scale<T>(p.a[0], row) * s0;
    }
}

__global__ void add_norm_generic(QrAddNormPost q, int d) {
    __shared__ float red[16];
    float ss = 0.f;
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        float s = q.u[i] + q.v[i];
        q.sum[i] = s;
        ss += s * s;
    }
    ss = block_sum(ss, red);
    float r = 1.f / sqrtf(ss / float(d) + q.eps);
    for (int i = threadIdx.x; i < d; i += blockDim.x) q.norm[i] = (q.sum[i] * r) * (q.weight[i] + q.offset);
}

template <WeightType T>
constexpr int elem() {
    return Elem<T>::E;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Chunks per lane supported by the fast kernel, and the row count per wave.
int pick_v(int need) {
    static const int vs[] = {1, 2, 4, 7, 8, 14, 16, 32};
    for (int v : vs)
        if (v >= need) return v;
    return 0;
}

// Rows per wave: 8 KiB of weights in flight per wave (V R = 8 chunks), one row
// from 8 chunks per lane on. Measured on the 0.8B shapes, one token, back to
// back: against 16 KiB per wave (R = 16 / V) a 3584 x 1024 matrix 5.07 -> 4.76
// us, 6144 x 1024 6.72 -> 6.05, 512 x 1024 3.88 -> 3.18, 1024 x 2048 4.48 ->
// 4.04; more waves, each with fewer loads ahead of its first FMA, start
// streaming sooner. Each row's sum is formed the same way for any R.
template <WeightType T, int V, int NB, int MODE>
int launch_vn(hipStream_t s, const GemvParams& p) {
    constexpr int R = V >= 8 ? 1 : 8 / V;
    GemvParams q = p;
    q.first[0] = 0;
    for (int i = 0; i < q.count; ++i) q.first[i + 1] = q.first[i] + int(ceil_div(q.rows[i], R));
    unsigned blocks = ceil_div(q.first[q.count], 4);
    hipLaunchKernelGGL((gemv_kernel<T, V, R, NB, MODE>), dim3(blocks), dim3(256), 0, s, q);
    return int(hipGetLastError());
}

template <WeightType T, int NB, int MODE>
int launch_v(hipStream_t s, const GemvParams& p, int v) {
    switch (v) {
    case 1: return launch_vn<T, 1, NB, MODE>(s, p);
    case 2: return launch_vn<T, 2, NB, MODE>(s, p);
    case 4: return launch_vn<T, 4, NB, MODE>(s, p);
    case 7: return launch_vn<T, 7, NB, MODE>(s, p);
    case 8: return launch_vn<T, 8, NB, MODE>(s, p);
    case 14: return launch_vn<T, 14, NB, MODE>(s, p);
    case 16: return launch_vn<T, 16, NB, MODE>(s, p);
    case 32: return launch_vn<T, 32, NB, MODE>(s, p);
    }
    return int(hipErrorInvalidValue);
}

template <WeightType T, int MODE>
int launch_nb(hipStream_t s, const GemvParams& p, int v, int nb) {
    if constexpr (MODE == kAddNorm) return launch_v<T, 1, MODE>(s, p, v);
    switch (nb) {
    case 1: return launch_v<T, 1, MODE>(s, p, v);
    case 2: return launch_v<T, 2, MODE>(s, p, v);
    case 3: return launch_v<T, 3, MODE>(s, p, v);
    case 4: return launch_v<T, 4, MODE>(s, p, v);
    default: return launch_v<T, 8, MODE>(s, p, v);  // never: callers split batches > 4
    }
}

// Whether the chunked kernel takes this matrix (16-byte rows and chunks).
template <WeightType T>
bool fast_ok(const void* a, int rows, int cols, const float* x) {
    constexpr int E = Elem<T>::E;
    if (cols % E != 0 || !aligned16(a) || !aligned16(x)) return false;
    if (T == WeightType::I8 && rows % 4 != 0) return false;
    return pick_v(int(ceil_div(cols / E, 64))) != 0;
}

template <WeightType T>
int group_t(hipStream_t s, const GemvItem* items, int n, const float* x, int cols, int batch) {
    bool fast = true;
    for (int i = 0; i < n; ++i) fast = fast && fast_ok<T>(items[i].a, items[i].rows, cols, x);
    if (!fast) {
        for (int i = 0; i < n; ++i) {
            GemvParams p{};
            p.a[0] = items[i].a;
            p.y[0] = items[i].y;
            p.rows[0] = items[i].rows;
            p.count = 1;
            p.x = x;
            p.cols = cols;
            hipLaunchKernelGGL((gemv_generic<T, kPlain>), dim3(unsigned(items[i].rows), unsigned(batch)), dim3(256), 0,
                               s, p);
            if (int e = int(hipGetLastError())) return e;
        }
        return 0;
    }
    const int v = pick_v(int(ceil_div(cols / Elem<T>::E, 64)));
    // Up to 4 tokens per pass (each pass reads the weights once).
    for (int t0 = 0; t0 < batch; t0 += 4) {
        const int nb = batch - t0 < 4 ? batch - t0 : 4;
        for (int i0 = 0; i0 < n; i0 += kGroupMax) {
            GemvParams p{};
            p.count = n - i0 < kGroupMax ? n - i0 : kGroupMax;
            for (int m = 0; m < p.count; ++m) {
                p.a[m] = items[i0 + m].a;
                p.y[m] = items[i0 + m].y + size_t(t0) * items[i0 + m].rows;
                p.rows[m] = items[i0 + m].rows;
            }
            p.x = x + size_t(t0) * cols;
            p.cols = cols;
            if (int e = launch_nb<T, kPlain>(s, p, v, nb)) return e;
        }
    }
    return 0;
}

template <WeightType T>
int glu_t(hipStream_t s, float* product, const void* gate, const void* up, const float* x, int rows, int cols,
          int batch) {
    GemvParams p{};
    p.a[0] = gate;
    p.up = up;
    p.y[0] = product;
    p.rows[0] = rows;
    p.count = 1;
    p.x = x;
    p.cols = cols;
    if (!(fast_ok<T>(gate, rows, cols, x) && fast_ok<T>(up, rows, cols, x))) {
        hipLaunchKernelGGL((gemv_generic<T, kGlu>), dim3(unsigned(rows), unsigned(batch)), dim3(256), 0, s, p);
        return int(hipGetLastError());
    }
    const int v = pick_v(int(ceil_div(cols / Elem<T>::E, 64)));
    for (int t0 = 0; t0 < batch; t0 += 4) {
        const int nb = batch - t0 < 4 ? batch - t0 : 4;
        p.x = x + size_t(t0) * cols;
        p.y[0] = product + size_t(t0) * rows;
        if (int e = launch_nb<T, kGlu>(s, p, v, nb)) return e;
    }
    return 0;
}

template <WeightType T>
int add_norm_t(hipStream_t s, float* y, const void* a, const float* x, int rows, int cols, const QrAddNormPost& post,
               unsigned* ticket) {
    GemvParams p{};
    p.a[0] = a;
    p.y[0] = y;
    p.rows[0] = rows;
    p.count = 1;
    p.x = x;
    p.cols = cols;
    p.post = post;
    p.ticket = ticket;
    if (!fast_ok<T>(a, rows, cols, x) || !ticket) {
        hipLaunchKernelGGL((gemv_generic<T, kPlain>), dim3(unsigned(rows), 1u), dim3(256), 0, s, p);
        if (int e = int(hipGetLastError())) return e;
        hipLaunchKernelGGL(add_norm_generic, dim3(1), dim3(256), 0, s, post, rows);
        return int(hipGetLastError());
    }
    return launch_nb<T, kAddNorm>(s, p, pick_v(int(ceil_div(cols / Elem<T>::E, 64))), 1);
}

}  // namespace

int gemv_group(hipStream_t s, WeightType t, const GemvItem* items, int n, const float* x, int cols, int batch) {
    switch (t) {
    case WeightType::F32: return group_t<WeightType::F32>(s, items, n, x, cols, batch);
    case WeightType::BF16: return group_t<WeightType::BF16>(s, items, n, x, cols, batch);
    case WeightType::I8: return group_t<WeightType::I8>(s, items, n, x, cols, batch);
    }
    return int(hipErrorInvalidValue);
}

int gemv_glu(hipStream_t s, WeightType t, float* product, const void* gate, const void* up, const float* x, int rows,
             int cols, int batch) {
    switch (t) {
    case WeightType::F32: return glu_t<WeightType::F32>(s, product, gate, up, x, rows, cols, batch);
    case WeightType::BF16: return glu_t<WeightType::BF16>(s, product, gate, up, x, rows, cols, batch);
    case WeightType::I8: return glu_t<WeightType::I8>(s, product, gate, up, x, rows, cols, batch);
    }
    return int(hipErrorInvalidValue);
}

int gemv_add_norm(hipStream_t s, WeightType t, float* y, const void* a, const float* x, int rows, int cols,
                  const QrAddNormPost& post, unsigned* ticket) {
    switch (t) {
    case WeightType::F32: return add_norm_t<WeightType::F32>(s, y, a, x, rows, cols, post, ticket);
    case WeightType::BF16: return add_norm_t<WeightType::BF16>(s, y, a, x, rows, cols, post, ticket);
    case WeightType::I8: return add_norm_t<WeightType::I8>(s, y, a, x, rows, cols, post, ticket);
    }
    return int(hipErrorInvalidValue);
}

}  // namespace qr
