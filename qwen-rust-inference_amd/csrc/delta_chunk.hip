// Chunked DeltaRule / DeltaRuleGated (ops 7 and 14) for prefill on gfx950:
// the recurrence of reference.h:149-170 (gates of reference.h:48-60),
// evaluated 64 tokens at a time in the WY / UT form so that the dense products
// run on fp32 MFMA (v_mfma_f32_32x32x2_f32) instead of one token per step.
//
// Per head, tokens t = 0..63 of a chunk, state S0 (dk x dv) entering it, log
// decay g_t, beta_t, and G_t = g_0 + ... + g_t:
//   S_t = e^{g_t} S_{t-1} + k_t d_t^T,   d_t = beta_t (v_t - e^{g_t} S_{t-1}^T k_t)
// unrolls to   d_t + sum_{s<t} A_ts d_s = beta_t v_t - beta_t e^{G_t} S0^T k_t,
// A_ts = beta_t e^{G_t - G_s} (k_t . k_s) for s < t, hence
//   D   = U - W S0,           U = (I + A)^{-1} (beta V),   W = (I + A)^{-1} (beta e^G K)
//   O   = (e^G Q) S0 + L D,   L_ts = e^{G_t - G_s} (q_t . k_s) for s <= t
//   S_C = e^{G_63} S0 + (e^{G_63 - G} K)^T D.
// Everything but S0 depends on the chunk's own inputs only:
// rule_chunk_prep_kernel builds U, -W, e^G Q, (e^{G_63-G} K)^T and L for all
// (chunk, head) pairs at once (the triangular solve is a forward substitution,
// one column per thread); rule_chunk_scan_kernel then walks the chunks in
// order, one block per (head, 32-column slice of S) with the slice in LDS.
// Tokens past the end of the last chunk are zero with g = 0 and beta = 0,
// which leaves D, O and S unchanged. G is summed in double so that
// G_t - G_s keeps its precision when G itself is large.
#include "common.h"

namespace qr {
namespace {

constexpr int kC = 64;     // tokens per chunk
constexpr int kD = 128;    // key_dim == value_dim
constexpr int kSlice = 32; // value columns per scan block
constexpr int kSlices = kD / kSlice;
// One (chunk, head) record, in floats: -W, U, e^G Q, (e^{G_63-G} K)^T, L, e^{G_63}.
constexpr int kW = 0, kU = kW + kC * kD, kQ = kU + kC * kD, kK = kQ + kC * kD, kL = kK + kD * kC,
              kG = kL + kC * kC, kRec = kG + 64;
constexpr int kGroupChunks = 64;  // chunks per prep + scan pair

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));

// A operand order of v_mfma_f32_32x32x2_f32 for a (32 x tiles) x (2 KH)
// matrix: in row tile `tile`, lane l feeds row l % 32 from the k-half l / 32,
// and step kk of the product uses k = (l / 32) KH + kk. float4 m of every
// lane (kk = 4m .. 4m+3) is stored as one contiguous 1 KiB run per wave.
template <int KH>
__device__ __forceinline__ int a_slot(int row, int k) {
    const int tile = row >> 5, l = (k / KH) * 32 + (row & 31), kk = k % KH;
    return tile * 64 * KH + (kk >> 2) * 256 + l * 4 + (kk & 3);
}
// Accumulator order of a 64 x 128 matrix in 32 x 32 tiles (row tile, column
// slice): register r of lane l holds row 8 (r / 4) + 4 (l / 32) + r % 4 and
// column l % 32; registers 4q .. 4q+3 of every lane are one 1 KiB run.
__device__ __forceinline__ int d_slot(int row, int col) {
    const int tile = row >> 5, lr = row & 31, q = lr >> 3, hl = (lr >> 2) & 1, e = lr & 3;
    const int js = col >> 5, l = hl * 32 + (col & 31);
    return ((tile * kSlices + js) * 4 + q) * 256 + l * 4 + e;
}
// Row of accumulator register r in lane half hl.
__device__ __forceinline__ int d_row(int r, int hl) { return 8 * (r >> 2) + 4 * hl + (r & 3); }

// LDS slots of the S slice (128 x 32) and of the D slice (64 x 32): the upper
// k-half is shifted by 32 banks, so the two lane halves of a B-operand read
// (rows kk and kk + KH) never meet in a bank.
__device__ __forceinline__ int s_lds(int row, int col) { return row * kSlice + col + (row >> 6) * kSlice; }
__device__ __forceinline__ int d_lds(int row, int col) { return row * kSlice + col + (row >> 5) * kSlice; }

__global__ __launch_bounds__(256) void rule_chunk_prep_kernel(Params a, int gated, int c0, float* scratch) {
    __shared__ float ks[kC][kD + 1], qs[kC][kD + 1];
    __shared__ float am[kC][kC + 4];
    __shared__ double gd[kC];
    __shared__ float bs[kC], eg[kC], el[kC];
    const int tid = threadIdx.x, h = blockIdx.y, c = c0 + int(blockIdx.x);
    const int kh = a.n[2], vh = a.n[3], tokens = a.n[4] > 0 ? a.n[4] : 1, stride = a.n[5];
    const int t0 = c * kC, n = min(kC, tokens - t0);
    float* rec = scratch + (size_t(blockIdx.x) * vh + h) * kRec;
    for (int e = tid; e < kC * kD; e += 256) {
        const int r = e / kD, i = e % kD;
        const size_t off = size_t(t0 + r) * vh * kD + size_t(h) * kD + i;
        ks[r][i] = r < n ? a.p[2][off] : 0.f;
        qs[r][i] = r < n ? a.p[1][off] : 0.f;
    }
    if (tid < kC) {  // wave 0: gates and the inclusive prefix of g
        float g = 0.f, b = 0.f;
        if (tid < n) {
            const int gi = (t0 + tid) * vh + h;
            if (gated) {
                g = -expf(a.p[7][vh + h]) * softplusf_(a.p[5][gi] + a.p[7][h]);
                b = sigmoidf_(a.p[6][gi]);
            } else {
                g = a.p[5][gi];
                b = a.p[6][gi];
            }
        }
        double G = g;
#pragma unroll
        for (int o = 1; o < kC; o <<= 1) {
            const double up = __shfl_up(G, o, kWave);
            if (tid >= o) G += up;
        }
        const double last = __shfl(G, kC - 1, kWave);
        gd[tid] = G;
        bs[tid] = b;
        eg[tid] = expf(float(G));
        el[tid] = expf(float(last - G));
    }
    __syncthreads();
    {  // Gram products: a 4 x 4 block of K K^T and Q K^T per thread
        const int tr = (tid >> 4) * 4, sc = (tid & 15) * 4;
        float kk[4][4] = {}, qk[4][4] = {};
        for (int i = 0; i < kD; ++i) {
            float kt[4], qt[4], kc[4];
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                kt[x] = ks[tr + x][i];
                qt[x] = qs[tr + x][i];
                kc[x] = ks[sc + x][i];
            }
#pragma unroll
            for (int x = 0; x < 4; ++x)
#pragma unroll
                for (int y = 0; y < 4; ++y) {
                    kk[x][y] = fmaf(kt[x], kc[y], kk[x][y]);
                    qk[x][y] = fmaf(qt[x], kc[y], qk[x][y]);
                }
        }
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int y = 0; y < 4; ++y) {
                const int t = tr + x, s = sc + y;
                const float e = s <= t ? expf(float(gd[t] - gd[s])) : 0.f;
                am[t][s] = s < t ? bs[t] * e * kk[x][y] : 0.f;
                rec[kL + a_slot<32>(t, s)] = e * qk[x][y];
            }
    }
    __syncthreads();
    for (int e = tid; e < kC * kD; e += 256) {
        const int t = e / kD, i = e % kD;
        rec[kQ + a_slot<64>(t, i)] = eg[t] * qs[t][i];
        rec[kK + a_slot<32>(i, t)] = el[t] * ks[t][i];
    }
    __syncthreads();
    // right-hand sides: beta e^G K in ks, beta V in qs
    for (int e = tid; e < kC * kD; e += 256) {
        const int t = e / kD, i = e % kD;
        ks[t][i] *= bs[t] * eg[t];
        qs[t][i] = t < n ? bs[t] * a.p[3][size_t(t0 + t) * stride + 2 * size_t(kh) * kD + size_t(h) * kD + i] : 0.f;
    }
    __syncthreads();
    {  // forward substitution (I + A) X = B, one column per thread: W (threads 0..127), U (128..255)
        const int col = tid & (kD - 1);
        const float* rhs = tid < kD ? &ks[0][col] : &qs[0][col];
        float x[kC];
#pragma unroll
        for (int t = 0; t < kC; ++t) {
            float r = rhs[t * (kD + 1)];
#pragma unroll
            for (int s = 0; s < t; ++s) r = fmaf(-am[t][s], x[s], r);
            x[t] = r;
            asm volatile("" ::: "memory");  // keep each row's LDS reads with its row
        }
        if (tid < kD) {
#pragma unroll
            for (int t = 0; t < kC; ++t) rec[kW + a_slot<64>(t, col)] = -x[t];
        } else {
#pragma unroll
            for (int t = 0; t < kC; ++t) rec[kU + d_slot(t, col)] = x[t];
        }
    }
    if (tid == 0) rec[kG] = eg[kC - 1];
}

__device__ __forceinline__ f16v mfma32(float x, float y, f16v acc) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc, 0, 0, 0);
}

// One block per (head, 32-column slice of S); waves 0, 1 own the D row tiles
// and waves 2, 3 the O row tiles of a chunk, and wave w updates S rows
// 32w .. 32w+31. Operands of the next chunk's first product are loaded while
// the current chunk's second product runs.
__global__ __launch_bounds__(256) void rule_chunk_scan_kernel(Params a, int c0, int chunks, const float* scratch) {
    __shared__ float sl[kD * kSlice + kSlice];
    __shared__ float dl[kC * kSlice + kSlice];
    const int h = int(blockIdx.x) / kSlices, js = int(blockIdx.x) % kSlices;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lc = l & 31, hl = l >> 5;
    const int vh = a.n[3], tokens = a.n[4] > 0 ? a.n[4] : 1;
    float* state = a.p[4] + size_t(h) * kD * kD + js * kSlice;
    for (int e = tid; e < kD * kSlice; e += 256) {
        const int r = e / kSlice, cc = e % kSlice;
        sl[s_lds(r, cc)] = state[size_t(r) * kD + cc];
    }
    // phase-1 operands of chunk c: -W (waves 0, 1) or e^G Q (waves 2, 3) rows of
    // tile w & 1, and U (waves 0, 1) in accumulator order
    const int first = w < 2 ? kW : kQ;
    auto load1 = [&](int c, f4v (&av)[16], f4v (&uv)[4]) {
        const float* rec = scratch + (size_t(c) * vh + h) * kRec;
        const f4v* A = reinterpret_cast<const f4v*>(rec + first + (w & 1) * 4096) + l;
#pragma unroll
        for (int m = 0; m < 16; ++m) av[m] = A[m * 64];
        const f4v* U = reinterpret_cast<const f4v*>(rec + kU + ((w & 1) * kSlices + js) * 1024) + l;
#pragma unroll
        for (int q = 0; q < 4; ++q) uv[q] = w < 2 ? U[q * 64] : f4v{0.f, 0.f, 0.f, 0.f};
    };
    f4v av[16], uv[4];
    load1(0, av, uv);
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
        const float* rec = scratch + (size_t(c) * vh + h) * kRec;
        const int t0 = (c0 + c) * kC;
        // phase-2 operands: L rows of tile w & 1 (waves 2, 3), (e^{G_63-G} K)^T rows of tile w
        f4v lv[8], kv[8];
        {
            const f4v* Lm = reinterpret_cast<const f4v*>(rec + kL + (w & 1) * 2048) + l;
            const f4v* K = reinterpret_cast<const f4v*>(rec + kK + w * 2048) + l;
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                lv[m] = w >= 2 ? Lm[m * 64] : f4v{0.f, 0.f, 0.f, 0.f};
                kv[m] = K[m * 64];
            }
        }
        const float decay = rec[kG];
        // phase 1: D = U - W S0 (waves 0, 1) or O = e^G Q S0 (waves 2, 3)
        f16v acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = uv[r >> 2][r & 3];
#pragma unroll
        for (int m = 0; m < 16; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = mfma32(av[m][e], sl[s_lds(hl * 64 + 4 * m + e, lc)], acc);
        const int R = (w & 1) * 32;
        if (w < 2) {
#pragma unroll
            for (int r = 0; r < 16; ++r) dl[d_lds(R + d_row(r, hl), lc)] = acc[r];
        }
        __syncthreads();
        if (c + 1 < chunks) load1(c + 1, av, uv);
        // phase 2: O += L D (waves 2, 3); S rows 32w.. = e^{G_63} S0 + (e^{G_63-G} K)^T D
        if (w >= 2) {
#pragma unroll
            for (int m = 0; m < 8; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc = mfma32(lv[m][e], dl[d_lds(hl * 32 + 4 * m + e, lc)], acc);
            float* out = a.p[0] + size_t(h) * kD + js * kSlice + lc;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t0 + R + d_row(r, hl);
                if (t < tokens) out[size_t(t) * vh * kD] = acc[r];
            }
        }
        f16v sacc;
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = decay * sl[s_lds(32 * w + d_row(r, hl), lc)];
#pragma unroll
        for (int m = 0; m < 8; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) sacc = mfma32(kv[m][e], dl[d_lds(hl * 32 + 4 * m + e, lc)], sacc);
#pragma unroll
        for (int r = 0; r < 16; ++r) sl[s_lds(32 * w + d_row(r, hl), lc)] = sacc[r];
        __syncthreads();
    }
    for (int e = tid; e < kD * kSlice; e += 256) {
        const int r = e / kSlice, cc = e % kSlice;
        state[size_t(r) * kD + cc] = sl[s_lds(r, cc)];
    }
}

}  // namespace

bool delta_rule_chunked_ok(const Params& a, int count) {
    const int tokens = a.n[4] > 0 ? a.n[4] : 1;
    return a.n[0] == kD && a.n[1] == kD && a.n[3] >= 1 && count == a.n[3] * kD && a.n[6] <= 0 &&
           tokens >= kChunkMinTokens;
}

size_t delta_rule_chunked_scratch(const Params& a) {
    const int tokens = a.n[4] > 0 ? a.n[4] : 1;
    const int chunks = int(ceil_div(tokens, kC));
    return size_t(chunks < kGroupChunks ? chunks : kGroupChunks) * size_t(a.n[3]) * kRec;
}

int run_delta_rule_chunked(hipStream_t s, bool gated, const Params& a, float* scratch, size_t len) {
    if (len < delta_rule_chunked_scratch(a)) return int(hipErrorInvalidValue);
    const int tokens = a.n[4] > 0 ? a.n[4] : 1, vh = a.n[3];
    const int chunks = int(ceil_div(tokens, kC));
    for (int c0 = 0; c0 < chunks; c0 += kGroupChunks) {
        const int group = chunks - c0 < kGroupChunks ? chunks - c0 : kGroupChunks;
        hipLaunchKernelGGL(rule_chunk_prep_kernel, dim3(unsigned(group), unsigned(vh)), dim3(256), 0, s, a,
                           gated ? 1 : 0, c0, scratch);
        if (hipError_t e = hipGetLastError()) return int(e);
        hipLaunchKernelGGL(rule_chunk_scan_kernel, dim3(unsigned(vh * kSlices)), dim3(256), 0, s, a, c0, group,
                           static_cast<const float*>(scratch));
        if (hipError_t e = hipGetLastError()) return int(e);
    }
    return 0;
}

}  // namespace qr
