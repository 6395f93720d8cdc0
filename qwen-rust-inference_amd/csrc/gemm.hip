// Prefill projections Y[batch, rows] = X[batch, cols] . A^T (batch >= 5) on
// gfx950, fp32 / BF16 / int8-per-row weights, fp32 accumulation.
//
// fp32 weights (the prefill of every config): BF16 MFMA
// (v_mfma_f32_32x32x16_bf16) on operands split into three BF16 parts each,
// which keeps fp32 accuracy (gemm_bf3_kernel below). A 128 (tokens) x 128
// (rows) output tile per 256-thread block, 2 x 2 waves of 64 x 64 (2 x 2 MFMA
// tiles each); K in steps of 32 through LDS; the next K step's global loads are
// in flight (registers) while the current one is multiplied.
// fp32 weights with at most 16 rows (the DeltaNet a / b projections):
// two such matrices per launch (x read once), up to 1024 columns, on fp32
// MFMA (gemm_ab_mfma_kernel) for cols % 16 == 0, else gemm_ab_kernel; wider
// rows: gemm_skinny_kernel (lanes over columns). BF16 and int8 weights of
// that shape (cols % 16 == 0) take gemm_ab_mfma_kernel too.
// Fewer 128 x 128 tiles than CUs: K split into chunks (partials + an ordered
// sum). The prefill GLU: gate and up in one MFMA kernel with silu(g) * u in
// the epilogue.
// BF16 / int8 weights (exact in BF16): the same kernel with one weight plane
// and three part products; int8 rows are scaled after the sum (scale *
// sum(q x), as the reference's qr_gemm_i8, native/rocm/bridge.cpp:620-653).
// Shapes the MFMA kernel does not take (cols % 4 != 0, unaligned operands):
// the LDS-tiled FMA kernel (64 x 64 tile, 4 x 4 outputs per thread).
#include "common.h"

namespace qr {
namespace {

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int MM = 128, MN = 128;

// ---- fp32 products on BF16 MFMA. Every fp32 operand is split into three
// BF16 parts, x = x0 + x1 + x2 (x0 = bf16(x), x1 = bf16(x - x0), x2 =
// bf16(x - x0 - x1); each residual is exact in fp32), and the six part
// products x_p y_q with p + q <= 2 are summed in fp32. The dropped products
// are below 2^-24 |x y| and every BF16 x BF16 product is exact, so a dot
// product keeps fp32 accuracy, while v_mfma_f32_32x32x16_bf16 does 16x the
// MACs per cycle of the fp32 MFMA (six of them per K step: 2.7x the rate).
// Per 32-deep K step each thread loads 4 float4 of X and of W, splits them and
// stores the three BF16 planes in LDS ([plane][row][k], rows of 40 BF16 = 80
// bytes, so the 16-byte operand reads of 8 consecutive lanes hit distinct
// banks). MFMA operands: lane l holds A[l % 32][8 (l / 32) + e] and
// B[8 (l / 32) + e][l % 32], e = 0..7; accumulator register r of lane l is
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
constexpr int B3K = 32, B3ROW = 40;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// One 32-deep K step of 128 rows (0-63 of `top` from top_r0, 64-127 of
// `bottom` from bottom_r0) into registers, as the raw words of the format:
// quad q of thread t is row (t + 256 q) / 8, k = 4 ((t + 256 q) % 8) (16 bytes
// of fp32, 8 of BF16 in .x/.y, 4 of int8 in .x; an int8 matrix's values follow
// its `rows` fp32 scales). k and k_end are multiples of 4 (cols % 4 == 0 and
// K chunks of whole 32-deep steps), so a quad is wholly inside or wholly
// outside [0, k_end). A quad outside the matrix is loaded from row 0, k 0 and
// its bit in `ok` cleared; b3_store writes it as zeros. Every quad is one
// unconditional load into its own registers and nothing reads them before
// b3_store, so the next step's loads stay in flight during the MFMAs.
template <WeightType T>
__device__ __forceinline__ void b3_load(const void* top, int top_r0, const void* bottom, int bottom_r0, int rows,
                                        int cols, int k0, int k_end, uint4 (&v)[4], unsigned& ok) {
    const int t = threadIdx.x;
    ok = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int f = t + 256 * q, rr = f >> 3, k = k0 + (f & 7) * 4;
        const void* m = rr < 64 ? top : bottom;
        const int r = (rr < 64 ? top_r0 : bottom_r0) + (rr & 63);
        const bool in = r < rows && k < k_end;
        ok |= unsigned(in) << q;
        const size_t e = in ? size_t(r) * cols + k : 0;
        if constexpr (T == WeightType::F32) {
            v[q] = *reinterpret_cast<const uint4*>(static_cast<const float*>(m) + e);
        } else if constexpr (T == WeightType::BF16) {
            const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(m) + e);
            v[q].x = w.x;
            v[q].y = w.y;
        } else {
            v[q].x = *reinterpret_cast<const unsigned*>(reinterpret_cast<const int8_t*>(static_cast<const float*>(m) + rows) + e);
        }
    }
}
// The loaded quads as fp32 (BF16 widened and int8 converted exactly; zeros
// where `ok` is clear), split into BF16 planes in LDS: three (x0, x1, x2) for
// fp32 or, for values exact in BF16 (BF16 and int8 weights), the one.
template <WeightType T>
__device__ __forceinline__ void b3_store(__bf16 (*lds)[128][B3ROW], const uint4 (&v)[4], unsigned ok) {
    constexpr int PLANES = T == WeightType::F32 ? 3 : 1;
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int f = t + 256 * q, rr = f >> 3, kq = (f & 7) * 4;
        f4v x;
        if constexpr (T == WeightType::F32) {
            x = f4v{__uint_as_float(v[q].x), __uint_as_float(v[q].y), __uint_as_float(v[q].z), __uint_as_float(v[q].w)};
        } else if constexpr (T == WeightType::BF16) {
            x = f4v{__uint_as_float(v[q].x << 16), __uint_as_float(v[q].x & 0xffff0000u), __uint_as_float(v[q].y << 16),
                    __uint_as_float(v[q].y & 0xffff0000u)};
        } else {
            const unsigned w = v[q].x;
            x = f4v{float(int(w << 24) >> 24), float(int(w << 16) >> 24), float(int(w << 8) >> 24), float(int(w) >> 24)};
        }
        if (!((ok >> q) & 1u)) x = f4v{0.f, 0.f, 0.f, 0.f};
        bf16x4 p0, p1, p2;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const __bf16 h0 = __bf16(x[e]);
            p0[e] = h0;
            if constexpr (PLANES == 3) {
                const float r1 = x[e] - float(h0);
                const __bf16 h1 = __bf16(r1);
                p1[e] = h1;
                p2[e] = __bf16(r1 - float(h1));
            }
        }
        *reinterpret_cast<bf16x4*>(&lds[0][rr][kq]) = p0;
        if constexpr (PLANES == 3) {
            *reinterpret_cast<bf16x4*>(&lds[1][rr][kq]) = p1;
            *reinterpret_cast<bf16x4*>(&lds[2][rr][kq]) = p2;
        }
    }
}

// GLU = false: Y = X A^T, a 128 x 128 tile per block (the wave's 64 x 64
// sub-tile is 2 x 2 MFMA tiles). GLU = true: product = silu(X G^T) * (X U^T)
// for 128 tokens x 64 rows, the weight tile being [64 gate rows | the same 64
// up rows]: the wave's sub-tile is 64 tokens x 32 rows of gate (j = 0) and of
// up (j = 1), so a gate value and its up partner sit in the same register of
// the same lane. blockIdx.z: the K split [z * kchunk, +kchunk); with more than
// one split the block writes its partial sums to y + z * batch * rows.
// T: fp32 weights take all six part products; BF16 and int8 weights are exact
// in BF16 (one plane), so x0 w, x1 w and x2 w; int8 sums are scaled after the
// sum (scale * sum(q x), the reference's qr_gemm_i8).
template <WeightType T, bool GLU>
__global__ __launch_bounds__(256) void gemm_bf3_kernel(float* y, const void* a, const void* a2, const float* x,
                                                       int rows, int cols, int batch, int kchunk) {
    constexpr int WP = T == WeightType::F32 ? 3 : 1;
    __shared__ __bf16 xs[3][128][B3ROW];
    __shared__ __bf16 ws[WP][128][B3ROW];
    constexpr int NT = GLU ? 64 : MN;  // output rows per block
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * (GLU ? 32 : 64);
    const int m0 = blockIdx.y * MM, n0 = blockIdx.x * NT;
    const int kbeg = int(blockIdx.z) * kchunk, kend = min(cols, kbeg + kchunk);
    float* out = y + size_t(blockIdx.z) * size_t(batch) * size_t(rows);
    const void* wbot = GLU ? a2 : a;
    const int wbot_r0 = GLU ? n0 : n0 + 64;
    f16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    uint4 xv[4], wv[4];
    unsigned xok, wok;
    b3_load<WeightType::F32>(x, m0, x, m0 + 64, batch, cols, kbeg, kend, xv, xok);
    b3_load<T>(a, n0, wbot, wbot_r0, rows, cols, kbeg, kend, wv, wok);
    b3_store<WeightType::F32>(xs, xv, xok);
    b3_store<T>(ws, wv, wok);
    __syncthreads();
    const int ar = lane & 31, ak = 8 * (lane >> 5);
    for (int k0 = kbeg; k0 < kend; k0 += B3K) {
        const bool more = k0 + B3K < kend;
        if (more) {  // next K step in flight while this one is multiplied
            b3_load<WeightType::F32>(x, m0, x, m0 + 64, batch, cols, k0 + B3K, kend, xv, xok);
            b3_load<T>(a, n0, wbot, wbot_r0, rows, cols, k0 + B3K, kend, wv, wok);
        }
#pragma unroll
        for (int ks = 0; ks < B3K / 16; ++ks) {
            bf16x8 av[2][3], bv[2][WP];
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int i = 0; i < 2; ++i) av[i][p] = *reinterpret_cast<const bf16x8*>(&xs[p][wm + 32 * i + ar][16 * ks + ak]);
#pragma unroll
            for (int p = 0; p < WP; ++p)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    bv[j][p] = *reinterpret_cast<const bf16x8*>(&ws[p][(GLU ? 64 * j + wn : wn + 32 * j) + ar][16 * ks + ak]);
            // the part products, smallest first; the four tiles interleaved
            constexpr int NPQ = WP == 3 ? 6 : 3;
#pragma unroll
            for (int pq = 0; pq < NPQ; ++pq) {
                constexpr int P[6] = {2, 1, 0, 1, 0, 0}, Q[6] = {0, 1, 2, 0, 1, 0};
                constexpr int P1[3] = {2, 1, 0};
                const int pa = WP == 3 ? P[pq] : P1[pq], pb = WP == 3 ? Q[pq] : 0;
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i][pa], bv[j][pb], acc[i][j], 0, 0, 0);
            }
        }
        __syncthreads();
        if (more) {
            b3_store<WeightType::F32>(xs, xv, xok);
            b3_store<T>(ws, wv, wok);
            __syncthreads();
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < (GLU ? 1 : 2); ++j) {
            const int n = n0 + wn + 32 * j + (lane & 31);
            if (n >= rows) continue;
            float sg = 1.f, su = 1.f;  // int8 row scales (gate / up, or the row's)
            if constexpr (T == WeightType::I8) {
                sg = static_cast<const float*>(a)[n];
                su = GLU ? static_cast<const float*>(a2)[n] : sg;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m >= batch) continue;
                if constexpr (GLU) {
                    const float g = T == WeightType::I8 ? sg * acc[i][0][r] : acc[i][0][r];
                    const float u = T == WeightType::I8 ? su * acc[i][1][r] : acc[i][1][r];
                    out[size_t(m) * rows + n] = siluf_(g) * u;
                } else {
                    out[size_t(m) * rows + n] = T == WeightType::I8 ? sg * acc[i][j][r] : acc[i][j][r];
                }
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
// idle, so K is cut into up to 16 chunks (multiples of the 32-deep step, at
// least two steps each) until there are about two blocks per CU. A block's K
// steps are latency-bound (one step of loads in flight), so a 128-token chunk
// wants many short K chunks: qkv 6144 x 1024 at 128 tokens, 48 tiles, takes
// 11 chunks of 3 steps.
int mfma_splits(int rows, int cols, int batch, int& kchunk) {
    const long tiles = long(ceil_div(rows, MN)) * long(ceil_div(batch, MM));
    int splits = 1;
    if (rows % 4 == 0)
        while (splits < 16 && tiles * splits < 2 * 256 && cols / (splits + 1) >= 2 * B3K) ++splits;
    kchunk = int(ceil_div(ceil_div(cols, splits), B3K)) * B3K;
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

// Up to two fp32 matrices of 32 rows together (the DeltaNet a / b
// projections, 16 rows each) over at most 1024 columns of the same x, in one
// launch that reads x once. Lane l of wave w holds row l % 32 (rows of matrix
// 1, then matrix 2) over columns [64 s, 64 s + 64), s = 2 w + l / 32, in
// registers for the whole launch; the block stages 8 token rows of x in LDS,
// every lane forms its 64-term dot for each token, and the 16 partials of a
// (token, row) are summed in slot order. Blocks stride over the 8-token groups.
constexpr int AB_ROWS = 32, AB_COLS = 1024, AB_TOK = 8, AB_SLOTS = AB_COLS / 64;
struct AbMats {
    float* y[2];
    const float* a[2];
    int rows[2];
};
__global__ __launch_bounds__(512) void gemm_ab_kernel(AbMats m, const float* x, int cols, int batch) {
    __shared__ f4v xs[AB_TOK][AB_COLS / 4];
    __shared__ float part[AB_TOK][AB_SLOTS][AB_ROWS + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 31, slot = 2 * wave + (lane >> 5);
    const int rows = m.rows[0] + m.rows[1];
    const int mi = r < m.rows[0] ? 0 : 1, rr = mi ? r - m.rows[0] : r;
    f4v wv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int k = 64 * slot + 4 * e;
        wv[e] = r < rows && k < cols ? *reinterpret_cast<const f4v*>(m.a[mi] + size_t(rr) * cols + k)
                                     : f4v{0.f, 0.f, 0.f, 0.f};
    }
    // the x rows of a round: this thread's float4 i = threadIdx.x + 512 j of
    // the round's AB_TOK x AB_COLS block, loaded one round ahead
    constexpr int XL = AB_TOK * AB_COLS / 4 / 512;
    auto load_x = [&](int g, f4v (&v)[XL]) {
#pragma unroll
        for (int j = 0; j < XL; ++j) {
            const int i = int(threadIdx.x) + 512 * j, t = i / (AB_COLS / 4), k = 4 * (i % (AB_COLS / 4));
            v[j] = g * AB_TOK + t < batch && k < cols
                       ? *reinterpret_cast<const f4v*>(x + size_t(g * AB_TOK + t) * cols + k)
                       : f4v{0.f, 0.f, 0.f, 0.f};
        }
    };
    f4v xn[XL];
    load_x(int(blockIdx.x), xn);
    for (int g = int(blockIdx.x); g * AB_TOK < batch; g += int(gridDim.x)) {
        const int t0 = g * AB_TOK;
#pragma unroll
        for (int j = 0; j < XL; ++j) {
            const int i = int(threadIdx.x) + 512 * j;
            xs[i / (AB_COLS / 4)][i % (AB_COLS / 4)] = xn[j];
        }
        __syncthreads();
        load_x(g + int(gridDim.x), xn);  // the next round's rows stream in while this one is summed
#pragma unroll
        for (int t = 0; t < AB_TOK; ++t) {
            float acc = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const f4v xv = xs[t][16 * slot + e];
                acc = fmaf(wv[e].x, xv.x, acc);
                acc = fmaf(wv[e].y, xv.y, acc);
                acc = fmaf(wv[e].z, xv.z, acc);
                acc = fmaf(wv[e].w, xv.w, acc);
            }
            part[t][slot][r] = acc;
        }
        __syncthreads();
        // no barrier after the sums: the next round writes xs only after every
        // wave has passed the barrier above (all xs reads done) and part only
        // after the next round's first barrier (all sums of this round done)
        if (int(threadIdx.x) < AB_TOK * AB_ROWS) {
            const int t = int(threadIdx.x) / AB_ROWS, o = int(threadIdx.x) % AB_ROWS;
            if (o < rows && t0 + t < batch) {
                float sum = 0.f;
                for (int j = 0; j < AB_SLOTS; ++j) sum += part[t][j][o];
                const int oi = o < m.rows[0] ? 0 : 1, orow = oi ? o - m.rows[0] : o;
                m.y[oi][size_t(t0 + t) * m.rows[oi] + orow] = sum;
            }
        }
    }
}

// The same two matrices (each up to 16 rows) on fp32 MFMA
// (v_mfma_f32_16x16x4_f32) when cols % 16 == 0: a block = 16 tokens x both
// matrices' rows, 8 waves, each with one accumulator tile per matrix (A = the
// weight rows, B = x^T) over the K steps m = w, w + 8, ... of 16 columns;
// step 4 m + e takes k = 16 m + 4 (lane / 16) + e, so every operand is one
// float4 load per m (at 1024 columns a wave's 8 loads per operand go out
// together, then its 64 MFMAs). The waves' partial tiles are added in wave
// order through LDS. The FMA kernel above streams x through LDS with one
// 16-byte LDS read per four FMAs; here the products run on the matrix cores.
// T: fp32, packed BF16 (values widened exactly to fp32 as they load, 8 bytes
// per 4 values) or int8 ([rows scales | values], 4 bytes per 4 values; each
// output scaled by its row's scale after the sum, as qr_gemm_i8).
constexpr int AB_WAVES = 8;
template <WeightType T>
__global__ __launch_bounds__(64 * AB_WAVES) void gemm_ab_mfma_kernel(AbMats m, const float* x, int cols, int batch) {
    __shared__ f4v part[AB_WAVES][2][64];
    const int lane = int(threadIdx.x & 63), w = int(threadIdx.x >> 6), lr = lane & 15, g = lane >> 4;
    const int tok = int(blockIdx.x) * 16 + lr, nm = cols / 16;
    const f4v z = {0.f, 0.f, 0.f, 0.f};
    f4v acc0 = z, acc1 = z;
    constexpr int B = 8;  // float4 of each operand in flight
    for (int mb = w; mb < nm; mb += AB_WAVES * B) {
        f4v xv[B], w0[B], w1[B];
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const int mm = mb + AB_WAVES * j, k = 16 * mm + 4 * g;
            const bool in = mm < nm;
            auto wload = [&](int mi) -> f4v {
                if (!(in && lr < m.rows[mi])) return z;
                if constexpr (T == WeightType::BF16) {
                    const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(m.a[mi]) +
                                                                    size_t(lr) * cols + k);
                    return f4v{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                               __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
                } else if constexpr (T == WeightType::I8) {
                    const unsigned v = *reinterpret_cast<const unsigned*>(
                        reinterpret_cast<const int8_t*>(m.a[mi] + m.rows[mi]) + size_t(lr) * cols + k);
                    return f4v{float(int(v << 24) >> 24), float(int(v << 16) >> 24), float(int(v << 8) >> 24),
                               float(int(v) >> 24)};
                } else {
                    return *reinterpret_cast<const f4v*>(m.a[mi] + size_t(lr) * cols + k);
                }
            };
            xv[j] = in && tok < batch ? *reinterpret_cast<const f4v*>(x + size_t(tok) * cols + k) : z;
            w0[j] = wload(0);
            w1[j] = wload(1);
        }
#pragma unroll
        for (int j = 0; j < B; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(w0[j][e], xv[j][e], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(w1[j][e], xv[j][e], acc1, 0, 0, 0);
            }
    }
    part[w][0][lane] = acc0;
    part[w][1][lane] = acc1;
    __syncthreads();
    if (w < 2 && tok < batch) {  // wave t sums matrix t: lane (lr, g) holds rows 4 g + r of token lr
        f4v sum = part[0][w][lane];
#pragma unroll
        for (int v = 1; v < AB_WAVES; ++v) sum += part[v][w][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (4 * g + r < m.rows[w]) {
                float v = sum[r];
                if constexpr (T == WeightType::I8) v = m.a[w][4 * g + r] * v;
                m.y[w][size_t(tok) * m.rows[w] + 4 * g + r] = v;
            }
    }
}

}  // namespace

bool gemm_preferred(WeightType, int, int, int batch) { return batch > 4; }

// The split-BF16 kernel loads 4 consecutive k of a row at once (16 bytes of
// X or fp32 weights, 8 of BF16, 4 of int8).
static bool mfma_ok(WeightType t, const void* a, const float* x, int cols) {
    return cols % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a) % (t == WeightType::F32 ? 16 : t == WeightType::BF16 ? 8 : 4) == 0;
}

size_t gemm_scratch(WeightType t, int rows, int cols, int batch) {
    if (t == WeightType::F32 && rows <= SK_ROWS) return 0;
    int kchunk;
    const int splits = mfma_splits(rows, cols, batch, kchunk);
    return splits > 1 ? size_t(splits) * size_t(rows) * size_t(batch) : 0;
}

bool gemm_ab_ok(WeightType t, const void* a, const float* x, int rows, int cols, int batch) {
    return (t == WeightType::F32 || cols % 16 == 0) && gemm_preferred(t, rows, cols, batch) && rows >= 1 &&
           rows <= AB_ROWS / 2 && cols <= AB_COLS && mfma_ok(t, a, x, cols);
}
int gemm_ab(hipStream_t s, float* y1, const float* a1, int rows1, float* y2, const float* a2, int rows2,
            const float* x, int cols, int batch, WeightType t) {
    if (rows1 < 1 || rows2 < 0 || rows1 + rows2 > AB_ROWS || (rows2 > 0 && (!y2 || !a2)) || cols % 4 != 0 ||
        cols > AB_COLS || batch < 1 || (t != WeightType::F32 && cols % 16 != 0))
        return int(hipErrorInvalidValue);
    const AbMats m{{y1, rows2 > 0 ? y2 : y1}, {a1, rows2 > 0 ? a2 : a1}, {rows1, rows2}};
    if (cols % 16 == 0 && rows1 <= 16 && rows2 <= 16) {
        const dim3 grid{unsigned(ceil_div(batch, 16))}, block{64u * AB_WAVES};
        if (t == WeightType::BF16)
            hipLaunchKernelGGL(gemm_ab_mfma_kernel<WeightType::BF16>, grid, block, 0, s, m, x, cols, batch);
        else if (t == WeightType::I8)
            hipLaunchKernelGGL(gemm_ab_mfma_kernel<WeightType::I8>, grid, block, 0, s, m, x, cols, batch);
        else
            hipLaunchKernelGGL(gemm_ab_mfma_kernel<WeightType::F32>, grid, block, 0, s, m, x, cols, batch);
        return int(hipGetLastError());
    }
    const int groups = int(ceil_div(batch, AB_TOK));
    hipLaunchKernelGGL(gemm_ab_kernel, dim3(unsigned(groups < 256 ? groups : 256)), dim3(512), 0, s, m, x, cols, batch);
    return int(hipGetLastError());
}

// The split-BF16 MFMA kernel over every weight format (with the K split), or
// -1 when the shape does not fit it.
template <WeightType T>
int gemm_bf3(hipStream_t s, float* y, const void* a, const float* x, int rows, int cols, int batch, float* work,
             size_t work_len) {
    int kchunk;
    const int splits = mfma_splits(rows, cols, batch, kchunk);
    const dim3 g(ceil_div(rows, MN), ceil_div(batch, MM), unsigned(splits));
    if (splits == 1) {
        hipLaunchKernelGGL((gemm_bf3_kernel<T, false>), g, dim3(256), 0, s, y, a, a, x, rows, cols, batch, kchunk);
        return int(hipGetLastError());
    }
    const size_t n = size_t(rows) * size_t(batch);
    if (!work || work_len < size_t(splits) * n) return int(hipErrorInvalidValue);
    hipLaunchKernelGGL((gemm_bf3_kernel<T, false>), g, dim3(256), 0, s, work, a, a, x, rows, cols, batch, kchunk);
    if (hipError_t e = hipGetLastError()) return int(e);
    hipLaunchKernelGGL(split_sum_kernel, dim3(ceil_div(long(n / 4), 256)), dim3(256), 0, s, y,
                       static_cast<const float*>(work), splits, n / 4);
    return int(hipGetLastError());
}

int gemm(hipStream_t s, WeightType t, float* y, const void* a, const float* x, int rows, int cols, int batch,
         float* work, size_t work_len) {
    dim3 grid(ceil_div(rows, BN), ceil_div(batch, BM));
    if (mfma_ok(t, a, x, cols)) {
        if (t != WeightType::F32 && rows <= AB_ROWS / 2 && cols <= AB_COLS && cols % 16 == 0)
            return gemm_ab(s, y, static_cast<const float*>(a), rows, nullptr, nullptr, 0, x, cols, batch, t);
        if (t == WeightType::F32 && rows <= SK_ROWS) {
            if (cols <= AB_COLS) return gemm_ab(s, y, static_cast<const float*>(a), rows, nullptr, nullptr, 0, x, cols, batch);
            hipLaunchKernelGGL(gemm_skinny_kernel, dim3(ceil_div(batch, 4 * SK_TOK)), dim3(256), 0, s, y,
                               static_cast<const float*>(a), x, rows, cols, batch);
            return int(hipGetLastError());
        }
        switch (t) {
        case WeightType::F32: return gemm_bf3<WeightType::F32>(s, y, a, x, rows, cols, batch, work, work_len);
        case WeightType::BF16: return gemm_bf3<WeightType::BF16>(s, y, a, x, rows, cols, batch, work, work_len);
        case WeightType::I8: return gemm_bf3<WeightType::I8>(s, y, a, x, rows, cols, batch, work, work_len);
        }
    }
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

bool gemm_glu_fused(WeightType t, const void* gate, const void* up, const float* x, int rows, int cols, int batch) {
    return gemm_preferred(t, rows, cols, batch) && mfma_ok(t, gate, x, cols) && mfma_ok(t, up, x, cols);
}

int gemm_glu(hipStream_t s, WeightType t, float* product, const void* gate, const void* up, const float* x, int rows,
             int cols, int batch) {
    const dim3 g(ceil_div(rows, 64), ceil_div(batch, MM), 1);
    switch (t) {
    case WeightType::F32:
        hipLaunchKernelGGL((gemm_bf3_kernel<WeightType::F32, true>), g, dim3(256), 0, s, product, gate, up, x, rows,
                           cols, batch, cols);
        break;
    case WeightType::BF16:
        hipLaunchKernelGGL((gemm_bf3_kernel<WeightType::BF16, true>), g, dim3(256), 0, s, product, gate, up, x, rows,
                           cols, batch, cols);
        break;
    case WeightType::I8:
        hipLaunchKernelGGL((gemm_bf3_kernel<WeightType::I8, true>), g, dim3(256), 0, s, product, gate, up, x, rows,
                           cols, batch, cols);
        break;
    }
    return int(hipGetLastError());
}

}  // namespace qr
