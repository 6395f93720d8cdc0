// Prefill projections of prepared fp32 matrices on gfx950: Y[M, N] = X[M, K]
// W[N, K]^T to fp32 accuracy, as BF16 MFMA over pre-split operand planes.
//
// The split: every fp32 value is x = x0 + x1 + x2 with x0 = bf16(x),
// x1 = bf16(x - x0), x2 = bf16(x - x0 - x1) (each residual exact in fp32).
// The product x w is the sum of the six part products x_p w_q with p + q <= 2
// (the three dropped ones are below 2^-24 |x w|), and every BF16 x BF16
// product is exact in fp32, so a dot product accumulated in fp32 keeps fp32
// accuracy.
//
// "P3" planes (layout in common.h): the three BF16 planes of a [rows, K]
// matrix in MFMA fragment order: the 32-row x 16-k fragment (rt, kt) of plane
// p is ONE contiguous KiB, lane l's 16 bytes at l * 16 being row 32 rt + l % 32,
// k 16 kt + 8 (l / 32) .. + 7: exactly the operand lane l of
// v_mfma_f32_32x32x16_bf16 holds. One row tile's K step of 32 (2 k tiles x 3
// planes) is 6 KiB contiguous.
//
// The GEMM (gemm_p3_kernel): a block tile of 128 tokens x 128 or 256 weight
// rows, 4 waves (2 x 2 waves of 64 x 64 or 64 x 128). K steps of 32 are copied
// global -> LDS by LDS DMA (global_load_lds_dwordx4: each instruction moves one
// fragment, 64 lanes x 16 bytes, straight into LDS) into two stages: the DMAs
// of step s + 1 are issued spread over step s's MFMAs (one every few) into the
// other stage and land while step s is multiplied. Per 16-deep k tile a wave
// reads 3 planes x its row tiles of
// X and of W and issues six MFMAs per (X tile, W tile) pair, so each operand
// read from LDS feeds six MFMAs: half the operand traffic of the same products
// laid out along K (a BF16 GEMM with K' = 6K reads a plane pair per product).
//
// Work split (make_plan): the tile grid is walked in whole rounds of 256
// blocks (one per CU); the tiles past the last whole round are split along K
// into chunks, so that round is as long as a chunk, not the whole K; their
// partial sums are added in chunk order by a second kernel (results do not
// depend on timing). Blocks of the whole rounds are dealt XCD-aware (the
// hardware deals blocks to the 8 XCDs round-robin): XCD x takes a contiguous
// range of the tile order, which walks groups of 8 tile rows column by column,
// so the blocks resident on one XCD share X rows and W rows in its L2.
//
// Prepared BF16 matrices ("P1": the one plane of a matrix whose values are
// exact in BF16, in the same fragment order) take the same kernels with one
// weight plane: three part products per step, x2 w, x1 w and x0 w, each
// operand read from LDS feeding three MFMAs.
//
// The prefill GLU (gemm_p3_glu_kernel): gate and up as one GEMM over planes
// that interleave them by 64 rows ([gate 64 | up 64] per 128 combined rows,
// p3_glu_interleave), so a wave's gate value and its up partner sit in the
// same register of the same lane; the epilogue writes silu(g) * u and the
// product's own P3 planes (the down projection's input), through LDS so the
// plane stores are 16 bytes wide.
#include "common.h"

namespace qr {
namespace {

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int FRAG = 1024;  // bytes of one 32 x 16 BF16 fragment
constexpr int BM = 128;     // block tile rows (tokens)

// A block tile of 128 tokens x (64 TNW) weight rows: 2 x 2 waves, each
// 64 x (32 TNW) = 2 x TNW MFMA tiles. One K step (32 deep) of one 32-row tile
// is 6 fragments of X (2 k tiles x 3 planes) and 2 WP of W (WP weight planes:
// 3, or 1 for BF16 weights); a stage holds the step's X fragments then its W
// fragments.
template <int TNW, int WP = 3>
struct Geo {
    static constexpr int BN = 64 * TNW;
    static constexpr int XRT = BM / 32, WRT = BN / 32;  // 32-row tiles per operand
    static constexpr int WF = 2 * WP;                   // W fragments per row tile and step
    static constexpr int FRAGS = 6 * XRT + WF * WRT;    // per stage
    static constexpr int STAGE = FRAGS * FRAG;
    static constexpr int DMA_PER_WAVE = FRAGS / 4;
    static_assert(FRAGS % 4 == 0, "the stage's DMAs split over 4 waves");
};

__device__ __forceinline__ void split3(float v, bf16x8 (&h)[3], int e) {
    const __bf16 h0 = __bf16(v);
    const float r1 = v - float(h0);
    const __bf16 h1 = __bf16(r1);
    h[0][e] = h0;
    h[1][e] = h1;
    h[2][e] = __bf16(r1 - float(h1));
}

// Waits until no vector memory operation of this wave is in flight (lgkmcnt
// and expcnt not waited).
__device__ __forceinline__ void vm_wait0() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Barrier that leaves DMA loads in flight: LDS operations done, then s_barrier.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// One fragment (1 KiB) global -> LDS: lane l's 16 bytes from src + 16 l land
// at LDS byte address dst + 16 l. Inline assembly, so that the compiler (which
// cannot tell which LDS bytes an LDS DMA writes) does not wait for every DMA
// in flight before each LDS read: the kernel orders them itself (vm_wait0,
// then the barrier that publishes a stage).
__device__ __forceinline__ void dma_frag(const char* src, unsigned dst, unsigned voff) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, %2" ::"v"(voff), "s"(dst), "s"(src)
                 : "memory", "m0");
}

// The tile grid of one launch and how its blocks share it (make_plan).
struct Plan {
    int M, N, kt;          // rows of X and of W (the GLU: combined rows), K / 16
    int tiles_m, tiles_n;  // 128-row tiles of X, BN-row tiles of W
    int full;              // tiles in whole-K blocks (the first of the grouped tile order)
    int full_grid;         // blocks of those: 8 ceil(full / 8)
    int rem;               // tiles split along K (the rest)
    int chunks, spc;       // K chunks of a split tile, 32-deep steps per chunk
    // int8 weights: the row scales (the GLU: gate's, and up's in scale_up),
    // applied after the sum; null otherwise
    const float* scale;
    const float* scale_up;
};

// Tile t of the grouped order: groups of 8 tile rows, column by column.
__device__ __forceinline__ void grouped(const Plan& p, int t, int& tm, int& tn) {
    constexpr int GM = 8;
    const int group = t / (GM * p.tiles_n), first = group * GM, gm = min(p.tiles_m - first, GM);
    const int in = t - group * GM * p.tiles_n;
    tm = first + in % gm;
    tn = in / gm;
}
// Block b's work: a whole tile (kc = -1) or chunk kc of split tile r. False
// for the spare blocks of the whole-tile range.
__device__ __forceinline__ bool block_work(const Plan& p, int b, int& tm, int& tn, int& kc, int& r) {
    if (b < p.full_grid) {
        const int per = p.full_grid / 8, t = (b & 7) * per + (b >> 3);
        if (t >= p.full) return false;
        grouped(p, t, tm, tn);
        kc = -1;
        r = 0;
        return true;
    }
    const int i = b - p.full_grid;
    r = i % p.rem;
    kc = i / p.rem;
    grouped(p, p.full + r, tm, tn);
    return true;
}

// One K step (two 16-deep k tiles) of the wave's 2 x TNW MFMA tiles from the
// stage at `st` (already offset by lane * 16). k tile 0's fragments are read
// first; k tile 1's reads go one each before the first MFMAs. With DMA, the
// wave's fragments of the next step (dma(i), i < DMA_PER_WAVE) are issued
// spread over the MFMA stream, one every few MFMAs: a burst of them after the
// barrier stalls the wave (the CU's vector memory path takes ~16 cycles per
// KiB, and the wave issues in order), while spread out they cost the MFMA
// stream nothing. sched_barrier(0) around each DMA keeps the scheduler from
// moving anything across it (it cannot classify the inline assembly).
template <int TNW, int WP, bool DMA, class F>
__device__ __forceinline__ void step_mfma(f16v (&acc)[2][TNW], const char* st, int wm, int wn, F&& dma) {
    using G = Geo<TNW, WP>;
    constexpr int NPQ = WP == 3 ? 6 : 3;              // part products per (X tile, W tile)
    constexpr int R = WP == 3 ? 3 * (2 + TNW) : 6 + TNW;  // fragment reads per k tile
    constexpr int MF = 2 * NPQ * TNW;                 // MFMAs per k tile
    constexpr int ND = G::DMA_PER_WAVE, EVERY = 2 * MF / ND;
    static_assert(R <= MF && EVERY >= 1 && ND * EVERY <= 2 * MF, "reads and DMAs fit the MFMA stream");
    bf16x8 a[2][2][3], b[2][TNW][WP];
    auto xfrag = [&](int k, int t, int pl) {
        return *reinterpret_cast<const bf16x8*>(st + ((2 * wm + t) * 6 + 3 * k + pl) * FRAG);
    };
    auto wfrag = [&](int k, int j, int pl) {
        return *reinterpret_cast<const bf16x8*>(st + (6 * G::XRT + (TNW * wn + j) * G::WF + WP * k + pl) * FRAG);
    };
    // read r of k tile k, in the order the products first use them: (x2, w0) (x1, w1) (x0, w2), or
    // with one weight plane (x2, w) then the x1 and x0 tiles
    auto read = [&](int k, int r) {
        if constexpr (WP == 3) {
            const int f = r / (2 + TNW), t = r % (2 + TNW);
            if (t < 2)
                a[k][t][2 - f] = xfrag(k, t, 2 - f);
            else
                b[k][t - 2][f] = wfrag(k, t - 2, f);
        } else if (r < 2 + TNW) {
            if (r < 2)
                a[k][r][2] = xfrag(k, r, 2);
            else
                b[k][r - 2][0] = wfrag(k, r - 2, 0);
        } else {
            const int rr = r - (2 + TNW), f = 1 + rr / 2, t = rr % 2;
            a[k][t][2 - f] = xfrag(k, t, 2 - f);
        }
    };
#pragma unroll
    for (int r = 0; r < R; ++r) read(0, r);
    // the part products, smallest first; the tiles interleaved
    constexpr int P[6] = {2, 1, 0, 1, 0, 0}, Q[6] = {0, 1, 2, 0, 1, 0};
    constexpr int P1[3] = {2, 1, 0};
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int pq = 0; pq < NPQ; ++pq)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j) {
                    const int n = ((k * NPQ + pq) * 2 + i) * TNW + j;
                    if (k == 0 && n < R) read(1, n);
                    const int pa = WP == 3 ? P[pq] : P1[pq], pb = WP == 3 ? Q[pq] : 0;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[k][i][pa], b[k][j][pb], acc[i][j], 0, 0, 0);
                    if (DMA && n % EVERY == EVERY / 2 && n / EVERY < ND) {
                        __builtin_amdgcn_sched_barrier(0);
                        dma(n / EVERY);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
}

// The K loop of one block: steps [s0, s0 + ns) of tile (tm, tn) into acc.
// Fragment c of a stage sits at c KiB: c < 6 XRT from X, else W; within an
// operand of F fragments per row tile and step (6, or 2 WP for W), row tile
// r = c' / F, then k tile and plane (c' % F = planes k + p), the order of the
// global layout, so fragment c of step s is at r rt_bytes + (F s + c' % F) KiB
// of its operand. Wave w moves fragments
// w DMA_PER_WAVE .. + DMA_PER_WAVE - 1: those of step s + 1 during step s's
// MFMAs, into the other stage (every wave finished reading it before the
// barrier of step s).
template <int TNW, int WP>
__device__ __forceinline__ void k_loop(f16v (&acc)[2][TNW], char* lds, const __bf16* xp, const __bf16* wp, int kt,
                                       int tm, int tn, int s0, int ns, int w, int lane) {
    using G = Geo<TNW, WP>;
    const size_t rt_x = size_t(kt) * 3 * FRAG, rt_w = size_t(kt) * WP * FRAG;  // one 32-row tile of a plane set
    const char* xb = reinterpret_cast<const char*>(xp) + size_t(tm) * G::XRT * rt_x + size_t(s0) * 6 * FRAG;
    const char* wb = reinterpret_cast<const char*>(wp) + size_t(tn) * G::WRT * rt_w + size_t(s0) * G::WF * FRAG;
    const unsigned lds0 = unsigned(reinterpret_cast<size_t>((__attribute__((address_space(3))) char*)lds));
    const unsigned voff = unsigned(lane) * 16u;
    const int wm = w & 1, wn = w >> 1;
    auto dma_one = [&](int s, int stage, int i) {
        const int c = w * G::DMA_PER_WAVE + i;
        const bool isw = c >= 6 * G::XRT;
        const int cc = isw ? c - 6 * G::XRT : c;
        const char* src;
        if constexpr (WP == 3)  // both operands 6 fragments per row tile and step
            src = (isw ? wb : xb) + size_t(cc / 6) * rt_x + size_t(6 * s + cc % 6) * FRAG;
        else
            src = isw ? wb + size_t(cc / G::WF) * rt_w + size_t(G::WF * s + cc % G::WF) * FRAG
                      : xb + size_t(cc / 6) * rt_x + size_t(6 * s + cc % 6) * FRAG;
        dma_frag(src, lds0 + unsigned(stage * G::STAGE + c * FRAG), voff);
    };
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
#pragma unroll
    for (int i = 0; i < G::DMA_PER_WAVE; ++i) dma_one(0, 0, i);
    int s = 0;
    for (; s + 1 < ns; ++s) {
        vm_wait0();     // this wave's fragments of step s landed
        lds_barrier();  // ... every wave's; and every wave is past its reads of step s - 1
        step_mfma<TNW, WP, true>(acc, lds + (s & 1) * G::STAGE + lane * 16, wm, wn,
                                 [&](int i) { dma_one(s + 1, (s + 1) & 1, i); });
    }
    vm_wait0();
    lds_barrier();
    step_mfma<TNW, WP, false>(acc, lds + (s & 1) * G::STAGE + lane * 16, wm, wn, [](int) {});
}

// Accumulator register e of lane l in MFMA tile (i, j) of wave (wm, wn): tile
// row 64 wm + 32 i + 8 (e / 4) + 4 (l / 32) + e % 4, column 32 (TNW wn + j) + l % 32.
__device__ __forceinline__ int acc_row(int wm, int i, int e, int lane) {
    return 64 * wm + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}

// Chunk kc of split tile r as raw sums: at (kc rem + r) BM BN of `work`, row-major BM x BN.
template <int TNW>
__device__ __forceinline__ void store_part(float* work, const Plan& p, int kc, int r, const f16v (&acc)[2][TNW],
                                           int wm, int wn, int lane) {
    constexpr int BN = Geo<TNW>::BN;
    float* part = work + (size_t(kc) * p.rem + r) * BM * BN;
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                part[acc_row(wm, i, e, lane) * BN + 32 * (TNW * wn + j) + (lane & 31)] = acc[i][j][e];
}

// Y = X W^T: whole tiles into y, chunks of split tiles into `work`. SC: each
// output column scaled by its weight row's p.scale after the sum (int8).
template <int TNW, int WP, bool SC = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WP == 3 ? 1 : 2, WP == 3 ? 1 : 2))) void gemm_p3_kernel(
    float* y, float* work, const __bf16* xp, const __bf16* wp, Plan p) {
    using G = Geo<TNW, WP>;
    __shared__ __attribute__((aligned(1024))) char lds[2 * G::STAGE];
    int tm, tn, kc, r;
    if (!block_work(p, int(blockIdx.x), tm, tn, kc, r)) return;
    const int lane = int(threadIdx.x) & 63, w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
    const int wm = w & 1, wn = w >> 1;
    const int s0 = kc < 0 ? 0 : kc * p.spc, ns = kc < 0 ? p.kt / 2 : min(p.kt / 2 - s0, p.spc);
    f16v acc[2][TNW];
    k_loop<TNW, WP>(acc, lds, xp, wp, p.kt, tm, tn, s0, ns, w, lane);
    if (kc >= 0) {
        store_part<TNW>(work, p, kc, r, acc, wm, wn, lane);
        return;
    }
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
        const int n = tn * G::BN + 32 * (TNW * wn + j) + (lane & 31);
        if (n >= p.N) continue;
        float sc = 1.f;
        if constexpr (SC) sc = p.scale[n];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = tm * BM + acc_row(wm, i, e, lane);
                if (m < p.M) y[size_t(m) * p.N + n] = SC ? sc * acc[i][j][e] : acc[i][j][e];
            }
    }
}

// The split tiles' chunks added in chunk order into y: one thread per 4
// consecutive columns of a tile row.
template <int BN>
__global__ __launch_bounds__(256) void p3_sum_kernel(float* y, const float* work, Plan p) {
    constexpr int per_tile = BM * BN / 4;
    const long i = long(blockIdx.x) * 256 + threadIdx.x;
    if (i >= long(p.rem) * per_tile) return;
    const int r = int(i / per_tile), e = int(i % per_tile) * 4, row = e / BN, col = e % BN;
    int tm, tn;
    grouped(p, p.full + r, tm, tn);
    const int m = tm * BM + row, n = tn * BN + col;
    if (m >= p.M) return;
    const size_t stride = size_t(p.rem) * BM * BN;
    const float* src = work + size_t(r) * BM * BN + e;
    f4v s = *reinterpret_cast<const f4v*>(src);
    for (int k = 1; k < p.chunks; ++k) s += *reinterpret_cast<const f4v*>(src + size_t(k) * stride);
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if (n + q < p.N) y[size_t(m) * p.N + n + q] = p.scale ? p.scale[n + q] * s[q] : s[q];
}

// ---- GLU: combined rows 128 g + [0, 64) are gate rows 64 g + .., 128 g +
// [64, 128) the up rows 64 g + .. (p3_glu_interleave). A 128 x 256 block tile
// covers gate / up rows 128 tn + [0, 128): wave wn's MFMA tiles j = 0, 1 are
// gate rows 128 tn + 64 wn + 32 j + .., tiles j = 2, 3 the same up rows.
// product[m][n] = silu(g) * u for n < I = N / 2, and (planes set) its P3
// planes with I / 16 k tiles.
__device__ __forceinline__ void glu_store8(float* product, __bf16* planes, int I, int m, int n, const float (&v)[8]) {
    *reinterpret_cast<f4v*>(product + size_t(m) * I + n) = f4v{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f4v*>(product + size_t(m) * I + n + 4) = f4v{v[4], v[5], v[6], v[7]};
    if (!planes) return;
    bf16x8 h[3];
#pragma unroll
    for (int e = 0; e < 8; ++e) split3(v[e], h, e);
#pragma unroll
    for (int q = 0; q < 3; ++q) *reinterpret_cast<bf16x8*>(planes + p3_index(m, n, q, I / 16)) = h[q];
}

template <int WP, bool SC = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WP == 3 ? 1 : 2, WP == 3 ? 1 : 2))) void gemm_p3_glu_kernel(
    float* product, __bf16* planes, float* work, const __bf16* xp, const __bf16* wp, Plan p) {
    using G = Geo<4, WP>;
    __shared__ __attribute__((aligned(1024))) char lds[2 * G::STAGE];
    int tm, tn, kc, r;
    if (!block_work(p, int(blockIdx.x), tm, tn, kc, r)) return;
    const int tid = int(threadIdx.x), lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w & 1, wn = w >> 1;
    const int s0 = kc < 0 ? 0 : kc * p.spc, ns = kc < 0 ? p.kt / 2 : min(p.kt / 2 - s0, p.spc);
    f16v acc[2][4];
    k_loop<4, WP>(acc, lds, xp, wp, p.kt, tm, tn, s0, ns, w, lane);
    if (kc >= 0) {  // raw gate / up sums of a chunk (p3_glu_sum_kernel finishes them)
        store_part<4>(work, p, kc, r, acc, wm, wn, lane);
        return;
    }
    // the product tile [128 tokens][128 columns] through LDS (row pitch 132
    // floats), then 8 consecutive columns per thread for 16-byte stores
    constexpr int PITCH = 132;
    static_assert(BM * PITCH * 4 <= 2 * G::STAGE, "product tile fits the stages");
    float* pt = reinterpret_cast<float*>(lds);
    lds_barrier();  // every wave past its last reads of the stages
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float sg = 1.f, su = 1.f;  // int8: the gate and up rows' scales of this product column
            if constexpr (SC) {
                const int n = tn * 128 + 64 * wn + 32 * j + (lane & 31);
                sg = p.scale[n];
                su = p.scale_up[n];
            }
#pragma unroll
            for (int e = 0; e < 16; ++e)
                pt[acc_row(wm, i, e, lane) * PITCH + 64 * wn + 32 * j + (lane & 31)] =
                    SC ? siluf_(sg * acc[i][j][e]) * (su * acc[i][j + 2][e]) : siluf_(acc[i][j][e]) * acc[i][j + 2][e];
        }
    lds_barrier();
    const int I = p.N / 2;
#pragma unroll
    for (int it = 0; it < BM * 16 / 256; ++it) {
        const int item = tid + 256 * it, row = item >> 4, c8 = (item & 15) * 8;
        const int m = tm * BM + row;
        if (m >= p.M) continue;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = pt[row * PITCH + c8 + e];
        glu_store8(product, planes, I, m, tn * 128 + c8, v);
    }
}

// The GLU's split tiles: gate and up chunks added in chunk order, then the
// product and its planes; one thread per 8 consecutive product columns.
__global__ __launch_bounds__(256) void p3_glu_sum_kernel(float* product, __bf16* planes, const float* work, Plan p) {
    constexpr int BN = 256, per_tile = BM * 16;
    const long i = long(blockIdx.x) * 256 + threadIdx.x;
    if (i >= long(p.rem) * per_tile) return;
    const int r = int(i / per_tile), row = int(i % per_tile) / 16, c8 = (int(i % per_tile) % 16) * 8;
    int tm, tn;
    grouped(p, p.full + r, tm, tn);
    const int m = tm * BM + row;
    if (m >= p.M) return;
    // product column c8 + e: wave wn = c8 / 64, gate tile column 128 wn + c8 % 64 + e, up 64 further
    const int gcol = 128 * (c8 >> 6) + (c8 & 63);
    const size_t stride = size_t(p.rem) * BM * BN;
    const float* src = work + size_t(r) * BM * BN + size_t(row) * BN;
    float g[8], u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        g[e] = src[gcol + e];
        u[e] = src[gcol + 64 + e];
    }
    for (int k = 1; k < p.chunks; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            g[e] += src[size_t(k) * stride + gcol + e];
            u[e] += src[size_t(k) * stride + gcol + 64 + e];
        }
    if (p.scale)  // int8: the rows' scales after the sums
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            g[e] = p.scale[tn * 128 + c8 + e] * g[e];
            u[e] = p.scale_up[tn * 128 + c8 + e] * u[e];
        }
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = siluf_(g[e]) * u[e];
    glu_store8(product, planes, p.N / 2, m, tn * 128 + c8, v);
}

// fp32 [rows, cols] -> P3 planes of p3_rows(rows) rows (the pad rows zero).
// Work item c is lane c % 64 of fragment c / 64 (32 rows x 16 k, row tile
// major): its 8 values (row 32 rt + lane % 32, k 16 kt + 8 (lane / 32)) are
// read as two 16-byte loads, and each wave writes whole 1 KiB fragments of
// the three planes, so the stores are contiguous (a row-major walk would
// scatter them 16 bytes per cache line).
__global__ __launch_bounds__(256) void p3_split_kernel(__bf16* out, const float* in, int rows, int cols, long chunks) {
    const int kt = cols / 16;
    for (long c = blockIdx.x * long(blockDim.x) + threadIdx.x; c < chunks; c += long(gridDim.x) * blockDim.x) {
        const long f = c >> 6;
        const int l = int(c & 63), rt = int(f / kt), kk = int(f % kt);
        const int r = 32 * rt + (l & 31), k = 16 * kk + 8 * (l >> 5);
        bf16x8 h[3];
        if (r < rows) {
            const f4v lo = *reinterpret_cast<const f4v*>(in + size_t(r) * cols + k);
            const f4v hi = *reinterpret_cast<const f4v*>(in + size_t(r) * cols + k + 4);
#pragma unroll
            for (int e = 0; e < 8; ++e) split3(e < 4 ? lo[e] : hi[e - 4], h, e);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) h[0][e] = h[1][e] = h[2][e] = __bf16(0.f);
        }
#pragma unroll
        for (int q = 0; q < 3; ++q) *reinterpret_cast<bf16x8*>(out + p3_index(r, k, q, kt)) = h[q];
    }
}

// Packed BF16 [rows, cols] (the reference's upload_bf16 words: element 2 i in
// the low half of word i) -> the one P1 plane of p3_rows(rows) rows (pad rows
// zero), in the fragment order of the P3 planes: work item c is lane c % 64 of
// fragment c / 64, 8 consecutive BF16 of one row, one 16-byte copy.
__global__ __launch_bounds__(256) void p1_from_bf16_kernel(__bf16* out, const uint16_t* in, int rows, int cols,
                                                           long chunks) {
    const int kt = cols / 16;
    for (long c = blockIdx.x * long(blockDim.x) + threadIdx.x; c < chunks; c += long(gridDim.x) * blockDim.x) {
        const long f = c >> 6;
        const int l = int(c & 63), rt = int(f / kt), kk = int(f % kt);
        const int r = 32 * rt + (l & 31), k = 16 * kk + 8 * (l >> 5);
        uint4 v = {0u, 0u, 0u, 0u};
        if (r < rows) v = *reinterpret_cast<const uint4*>(in + size_t(r) * cols + k);
        *reinterpret_cast<uint4*>(out + size_t(c) * 8) = v;
    }
}

// The int8 values of a [rows fp32 scales | rows x cols int8] matrix (the
// reference's upload_int8) -> their one P1 plane (integers of magnitude <= 128
// are exact in BF16; the scales stay in the matrix and are applied after the
// sum): 8 values, one 16-byte store, per work item as p1_from_bf16_kernel.
__global__ __launch_bounds__(256) void p1_from_i8_kernel(__bf16* out, const int8_t* in, int rows, int cols,
                                                         long chunks) {
    typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
    const int kt = cols / 16;
    for (long c = blockIdx.x * long(blockDim.x) + threadIdx.x; c < chunks; c += long(gridDim.x) * blockDim.x) {
        const long f = c >> 6;
        const int l = int(c & 63), rt = int(f / kt), kk = int(f % kt);
        const int r = 32 * rt + (l & 31), k = 16 * kk + 8 * (l >> 5);
        bf16x8v h;
        uint2 v = {0u, 0u};
        if (r < rows) v = *reinterpret_cast<const uint2*>(in + size_t(r) * cols + k);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const unsigned w = e < 4 ? v.x : v.y;
            h[e] = __bf16(float(int(w << (24 - 8 * (e & 3))) >> 24));
        }
        *reinterpret_cast<bf16x8v*>(out + size_t(c) * 8) = h;
    }
}

// The GLU's combined planes from gate's and up's (each rows x cols, rows %
// 128 == 0, 3 planes or BF16's 1): combined 32-row tile 4 g + t is gate tile
// 2 g + t (t < 2), else up tile 2 g + t - 2; a tile is contiguous, so this is
// a copy, 16 bytes per thread.
__global__ __launch_bounds__(256) void p3_glu_interleave_kernel(__bf16* out, const __bf16* gate, const __bf16* up,
                                                                int tiles, size_t tile_elems) {
    const size_t per_tile = tile_elems / 8, total = size_t(tiles) * per_tile;
    for (size_t c = blockIdx.x * size_t(blockDim.x) + threadIdx.x; c < total; c += size_t(gridDim.x) * blockDim.x) {
        const size_t t = c / per_tile, e = (c % per_tile) * 8;
        const size_t g = t / 4, q = t % 4;
        const __bf16* src = (q < 2 ? gate : up) + (2 * g + (q & 1)) * tile_elems + e;
        *reinterpret_cast<bf16x8*>(out + t * tile_elems + e) = *reinterpret_cast<const bf16x8*>(src);
    }
}

// Microseconds of one 32-deep K step of a 128 x bn block tile at the rate the
// kernels reach on the prefill shapes (0.8B model, 2644 tokens); one weight
// plane: half the MFMAs.
double step_us(int bn, int wp) { return (bn == 256 ? 2.9 : 1.66) * (wp == 3 ? 1.0 : 1.1); }
// Blocks per round: one per CU (three weight planes: 144 KiB of LDS), two
// (one plane: 80 KiB each).
int round_blocks(int wp) { return wp == 3 ? 256 : 512; }

// The plan of an M x N (x K) product with bn-row W tiles: whole rounds of 256
// blocks take whole tiles; the tiles past them (all, when there are fewer than
// 256) are split into K chunks when that is estimated faster: the split
// round's time, plus the partials' sum (their bytes at ~4 TB/s plus ~4 us).
Plan make_plan(int M, int N, int K, int bn, int wp) {
    Plan p{};
    p.M = M;
    p.N = N;
    p.kt = K / 16;
    p.tiles_m = int(ceil_div(M, BM));
    p.tiles_n = int(ceil_div(N, bn));
    const int tiles = p.tiles_m * p.tiles_n, steps = K / 32;
    const int slots = round_blocks(wp), whole = tiles / slots, rest = tiles - slots * whole;
    int best_c = 1;
    double best = double(ceil_div(tiles, slots)) * steps * step_us(bn, wp);
    for (int c = 2; c <= 8 && steps / c >= 4 && rest > 0; ++c) {
        const double t =
            (double(whole) * steps + double(ceil_div(long(rest) * c, slots)) * ceil_div(steps, c)) * step_us(bn, wp) +
            double(rest) * BM * bn * 4.0 * (c + 1) / 4e6 + 4.0;
        if (t < best) {
            best = t;
            best_c = c;
        }
    }
    if (best_c == 1) {
        p.full = tiles;
        p.rem = 0;
        p.chunks = 1;
        p.spc = steps;
    } else {
        p.full = slots * whole;
        p.rem = rest;
        p.spc = int(ceil_div(steps, best_c));
        p.chunks = int(ceil_div(steps, p.spc));
    }
    p.full_grid = 8 * int(ceil_div(p.full, 8));
    return p;
}

// The estimated time of a plan.
double plan_us(const Plan& p, int K, int bn, int wp) {
    const int slots = round_blocks(wp);
    return (double(ceil_div(p.full, slots)) * (K / 32) + double(ceil_div(long(p.rem) * p.chunks, slots)) * p.spc) *
               step_us(bn, wp) +
           (p.rem ? double(p.rem) * BM * bn * 4.0 * (p.chunks + 1) / 4e6 + 4.0 : 0.0);
}

// The W tile width of a plain product: 256 rows unless 128-row tiles are
// estimated faster.
int plain_bn(int M, int N, int K, int wp) {
    return plan_us(make_plan(M, N, K, 128, wp), K, 128, wp) < plan_us(make_plan(M, N, K, 256, wp), K, 256, wp) ? 128
                                                                                                              : 256;
}

size_t scratch_of(const Plan& p, int bn) { return size_t(p.rem) * size_t(p.chunks) * BM * size_t(bn); }

template <int WP, bool SC>
void launch_gemm(hipStream_t s, int bn, dim3 grid, float* y, float* work, const __bf16* xp, const __bf16* wp,
                 const Plan& p) {
    if (bn == 256)
        hipLaunchKernelGGL((gemm_p3_kernel<4, WP, SC>), grid, dim3(256), 0, s, y, work, xp, wp, p);
    else
        hipLaunchKernelGGL((gemm_p3_kernel<2, WP, SC>), grid, dim3(256), 0, s, y, work, xp, wp, p);
}

}  // namespace

size_t p3_elements(int rows, int cols) { return size_t(p3_rows(rows)) * size_t(cols) * 3; }
size_t p1_elements(int rows, int cols) { return size_t(p3_rows(rows)) * size_t(cols); }

int p3_split(hipStream_t s, __bf16* out, const float* in, int rows, int cols) {
    if (rows < 1 || !p3_cols_ok(cols) || reinterpret_cast<uintptr_t>(in) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(out) % 16 != 0)
        return int(hipErrorInvalidValue);
    const long chunks = long(p3_rows(rows)) * (cols / 8), blocks = (chunks + 255) / 256;
    hipLaunchKernelGGL(p3_split_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, s, out, in,
                       rows, cols, chunks);
    return int(hipGetLastError());
}

int p1_from_bf16(hipStream_t s, __bf16* out, const void* packed, int rows, int cols) {
    if (rows < 1 || !p3_cols_ok(cols) || reinterpret_cast<uintptr_t>(packed) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(out) % 16 != 0)
        return int(hipErrorInvalidValue);
    const long chunks = long(p3_rows(rows)) * (cols / 8), blocks = (chunks + 255) / 256;
    hipLaunchKernelGGL(p1_from_bf16_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, s, out,
                       static_cast<const uint16_t*>(packed), rows, cols, chunks);
    return int(hipGetLastError());
}

int p1_from_i8(hipStream_t s, __bf16* out, const void* packed, int rows, int cols) {
    const int8_t* values = reinterpret_cast<const int8_t*>(static_cast<const float*>(packed) + rows);
    if (rows < 1 || !p3_cols_ok(cols) || reinterpret_cast<uintptr_t>(values) % 8 != 0 ||
        reinterpret_cast<uintptr_t>(out) % 16 != 0)
        return int(hipErrorInvalidValue);
    const long chunks = long(p3_rows(rows)) * (cols / 8), blocks = (chunks + 255) / 256;
    hipLaunchKernelGGL(p1_from_i8_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, s, out,
                       values, rows, cols, chunks);
    return int(hipGetLastError());
}

int p3_glu_interleave(hipStream_t s, __bf16* out, const __bf16* gate, const __bf16* up, int rows, int cols,
                      int planes) {
    if (rows < 128 || rows % 128 != 0 || !p3_cols_ok(cols) || (planes != 3 && planes != 1) ||
        ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up)) % 16))
        return int(hipErrorInvalidValue);
    const size_t tile = size_t(32) * size_t(cols) * size_t(planes);
    const int tiles = 2 * rows / 32;
    const size_t total = size_t(tiles) * tile / 8, blocks = (total + 255) / 256;
    hipLaunchKernelGGL(p3_glu_interleave_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, s,
                       out, gate, up, tiles, tile);
    return int(hipGetLastError());
}

size_t p3_gemm_scratch(int M, int N, int K, int wplanes) {
    if (M < 1 || N < 1 || !p3_cols_ok(K)) return 0;
    const int bn = plain_bn(M, N, K, wplanes);
    return scratch_of(make_plan(M, N, K, bn, wplanes), bn);
}
size_t p3_glu_scratch(int M, int rows, int K, int wplanes) {
    if (M < 1 || rows < 1 || !p3_cols_ok(K)) return 0;
    return scratch_of(make_plan(M, 2 * rows, K, 256, wplanes), 256);
}

int p3_gemm(hipStream_t s, float* y, const __bf16* xp, const __bf16* wp, int M, int N, int K, float* work,
            size_t work_len, int wplanes, const float* scale) {
    if (M < 1 || N < 1 || !p3_cols_ok(K) || (wplanes != 3 && wplanes != 1) || (scale && wplanes != 1) ||
        ((reinterpret_cast<uintptr_t>(xp) | reinterpret_cast<uintptr_t>(wp)) % 16))
        return int(hipErrorInvalidValue);
    const int bn = plain_bn(M, N, K, wplanes);
    Plan p = make_plan(M, N, K, bn, wplanes);
    p.scale = scale;
    if (p.rem > 0 && (!work || work_len < scratch_of(p, bn))) return int(hipErrorInvalidValue);
    const dim3 grid{unsigned(p.full_grid + p.rem * p.chunks)}, block{256u};
    if (wplanes == 3)
        launch_gemm<3, false>(s, bn, grid, y, work, xp, wp, p);
    else if (scale)
        launch_gemm<1, true>(s, bn, grid, y, work, xp, wp, p);
    else
        launch_gemm<1, false>(s, bn, grid, y, work, xp, wp, p);
    if (p.rem > 0) {
        const long n = long(p.rem) * BM * bn / 4;
        if (bn == 256)
            hipLaunchKernelGGL(p3_sum_kernel<256>, dim3(unsigned((n + 255) / 256)), block, 0, s, y, work, p);
        else
            hipLaunchKernelGGL(p3_sum_kernel<128>, dim3(unsigned((n + 255) / 256)), block, 0, s, y, work, p);
    }
    return int(hipGetLastError());
}

int p3_gemm_glu(hipStream_t s, float* product, __bf16* planes, const __bf16* xp, const __bf16* wglu, int M, int rows,
                int K, float* work, size_t work_len, int wplanes, const float* scale_gate, const float* scale_up) {
    if (M < 1 || rows < 128 || rows % 128 != 0 || !p3_cols_ok(K) || (wplanes != 3 && wplanes != 1) ||
        (!scale_gate != !scale_up) || (scale_gate && wplanes != 1) ||
        ((reinterpret_cast<uintptr_t>(xp) | reinterpret_cast<uintptr_t>(wglu) | reinterpret_cast<uintptr_t>(product) |
          reinterpret_cast<uintptr_t>(planes)) % 16))
        return int(hipErrorInvalidValue);
    Plan p = make_plan(M, 2 * rows, K, 256, wplanes);
    p.scale = scale_gate;
    p.scale_up = scale_up;
    if (p.rem > 0 && (!work || work_len < scratch_of(p, 256))) return int(hipErrorInvalidValue);
    const dim3 grid{unsigned(p.full_grid + p.rem * p.chunks)}, block{256u};
    if (wplanes == 3)
        hipLaunchKernelGGL((gemm_p3_glu_kernel<3, false>), grid, block, 0, s, product, planes, work, xp, wglu, p);
    else if (scale_gate)
        hipLaunchKernelGGL((gemm_p3_glu_kernel<1, true>), grid, block, 0, s, product, planes, work, xp, wglu, p);
    else
        hipLaunchKernelGGL((gemm_p3_glu_kernel<1, false>), grid, block, 0, s, product, planes, work, xp, wglu, p);
    if (p.rem > 0) {
        const long n = long(p.rem) * BM * 16;
        hipLaunchKernelGGL(p3_glu_sum_kernel, dim3(unsigned((n + 255) / 256)), block, 0, s, product, planes, work, p);
    }
    return int(hipGetLastError());
}

}  // namespace qr
