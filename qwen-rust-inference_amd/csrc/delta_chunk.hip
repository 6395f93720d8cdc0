// Chunked DeltaRule / DeltaRuleGated (ops 7 and 14) for prefill on gfx950:
// the recurrence of reference.h:149-170 (gates of reference.h:48-60),
// evaluated 64 tokens at a time in the WY / UT form so that the dense products
// run on fp32 MFMA (v_mfma_f32_16x16x4_f32) instead of one token per step.
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
// (chunk, head) pairs of a group of chunks at once (8 waves; the triangular
// solve by 16-row blocks on MFMA with the inverses of the diagonal blocks);
// rule_chunk_scan_kernel then walks the group's chunks in order, one block per
// (head, 16-column slice of S) with the slice in LDS. With several groups,
// rule_chunk_scan_prep_kernel scans group g on half the CUs while the other
// half makes group g + 1's records (two record buffers).
// Tokens past the end of the last chunk are zero with g = 0 and beta = 0,
// which leaves D, O and S unchanged. G is summed in double so that
// G_t - G_s keeps its precision when G itself is large.
#include "common.h"

namespace qr {
namespace {

constexpr int kC = 64;     // tokens per chunk
constexpr int kD = 128;    // key_dim == value_dim
constexpr int kSlice = 16; // value columns per scan block
constexpr int kSlices = kD / kSlice;
// One (chunk, head) record, in floats: -W, U, e^G Q, (e^{G_63-G} K)^T, L, e^{G_63}.
constexpr int kW = 0, kU = kW + kC * kD, kQ = kU + kC * kD, kK = kQ + kC * kD, kL = kK + kD * kC,
              kG = kL + kC * kC, kRec = kG + 64;

typedef float f4v __attribute__((ext_vector_type(4)));

// Record layouts, for v_mfma_f32_16x16x4_f32 (lane l: A[i = l % 16][k = l / 16],
// B[k = l / 16][j = l % 16], accumulator register r: row 4 (l / 16) + r,
// column l % 16). Step s of a product over K uses k = 4 s + (l / 16), so the
// B rows a step reads are 4 consecutive rows (conflict-free in a [rows][16]
// LDS array).
// A operand of a (16 x tiles) x K matrix: float4 m of lane l in row tile
// `tile` holds row 16 tile + l % 16 at k = 16 m + l / 16 + 4 e (e = 0..3),
// every lane's float4 m one contiguous 1 KiB run. f4 index of (tile, m, l):
// tile * K + m * 64 + l.
// U in accumulator order: f4 (tile, js, l) holds rows 16 tile + 4 (l / 16) + e
// of column 16 js + l % 16; f4 index (tile * kSlices + js) * 64 + l.

constexpr int kPrep = 512;              // threads of a prep block (8 waves)
constexpr int kPrepLoads = kC * kD / 4 / kPrep;  // float4 of q (of k, of V) per thread

struct PrepLds {
    // row stride 132 (4 mod 64 banks): the Gram products' MFMA operand reads
    // (16 rows x 4 interleaved k per step) hit 64 distinct banks
    float ks[kC][kD + 4], qs[kC][kD + 4];
    // am holds A transposed: am[s][t] = A_ts (s < t), so the solve's column
    // sweeps read rows
    float am[kC][kC + 4], lm[kC][kC + 4];
    // inverses of the four 16 x 16 diagonal blocks of I + A: li[i][t][s] = ((I + A)_ii^-1)_ts
    float li[kC / 16][16][16];
    double gd[kC];
    float bs[kC], eg[kC], el[kC];
};

// The record of chunk c0 + xi of head h, into slot xi of `scratch`; every
// thread of a kPrep-thread block takes part.
__device__ __forceinline__ void prep_task(const Params& a, int gated, int qkn, int c0, float* scratch, int xi, int h,
                                          PrepLds& P) {
    auto& ks = P.ks;
    auto& qs = P.qs;
    auto& am = P.am;
    auto& lm = P.lm;
    auto& li = P.li;
    auto& gd = P.gd;
    auto& bs = P.bs;
    auto& eg = P.eg;
    auto& el = P.el;
    const int tid = threadIdx.x, c = c0 + xi;
    const int kh = a.n[2], vh = a.n[3], tokens = a.n[4] > 0 ? a.n[4] : 1, stride = a.n[5];
    const int t0 = c * kC, n = min(kC, tokens - t0);
    float* rec = scratch + (size_t(xi) * vh + h) * kRec;
    f4v* rec4 = reinterpret_cast<f4v*>(rec);
    // Every global input of the block is requested up front: the gate inputs
    // (wave 0), q and k rows, and the V rows, held in registers until the
    // right-hand sides are formed, so no later phase waits on a load.
    float ga = 0.f, gb = 0.f, gdt = 0.f, galog = 0.f;
    if (tid < n) {
        const int gi = (t0 + tid) * vh + h;
        ga = a.p[5][gi];
        gb = a.p[6][gi];
        if (gated) {
            gdt = a.p[7][h];
            galog = a.p[7][vh + h];
        }
    }
    f4v vv[kPrepLoads];
    {  // q and k rows: every thread's float4 loads in flight together
        f4v kv[kPrepLoads], qv[kPrepLoads];
        // qkn: the rows are the convolution's q and k of the head's key head,
        // L2-normalised here as DeltaQk does (reference.h:134-143) and stored
        // to the query / key outputs too; else DeltaQk's outputs
        const int hk = qkn ? h / (vh / kh) : 0;  // the host checks kh >= 1 and vh % kh == 0 for qkn
        const float* qsrc = qkn ? a.p[3] + size_t(hk) * kD : a.p[1] + size_t(h) * kD;
        const float* ksrc = qkn ? a.p[3] + size_t(kh + hk) * kD : a.p[2] + size_t(h) * kD;
        const size_t rs = qkn ? size_t(stride) : size_t(vh) * kD;
#pragma unroll
        for (int j = 0; j < kPrepLoads; ++j) {
            const int e = tid + kPrep * j, r = e >> 5, i = (e & 31) * 4;
            const size_t off = size_t(t0 + r) * rs + i;
            const f4v z = {0.f, 0.f, 0.f, 0.f};
            kv[j] = r < n ? *reinterpret_cast<const f4v*>(ksrc + off) : z;
            qv[j] = r < n ? *reinterpret_cast<const f4v*>(qsrc + off) : z;
        }
#pragma unroll
        for (int j = 0; j < kPrepLoads; ++j) {
            const int e = tid + kPrep * j, t = e >> 5, i = (e & 31) * 4;
            const f4v z = {0.f, 0.f, 0.f, 0.f};
            vv[j] = t < n ? *reinterpret_cast<const f4v*>(a.p[3] + size_t(t0 + t) * stride + 2 * size_t(kh) * kD +
                                                          size_t(h) * kD + i)
                          : z;
        }
        if (qkn) {  // a row is one half-wave (32 lanes x 4 elements): its sums by xor shuffles
            const float sd = sqrtf(float(kD));
#pragma unroll
            for (int j = 0; j < kPrepLoads; ++j) {
                const int e = tid + kPrep * j, r = e >> 5, i = (e & 31) * 4;
                float sq = qv[j].x * qv[j].x + qv[j].y * qv[j].y + qv[j].z * qv[j].z + qv[j].w * qv[j].w;
                float sk = kv[j].x * kv[j].x + kv[j].y * kv[j].y + kv[j].z * kv[j].z + kv[j].w * kv[j].w;
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) {
                    sq += __shfl_xor(sq, o, kWave);
                    sk += __shfl_xor(sk, o, kWave);
                }
                const float rq = 1.f / sqrtf(sq + 1e-6f), rk = 1.f / sqrtf(sk + 1e-6f);
                qv[j] = f4v{(qv[j].x * rq) / sd, (qv[j].y * rq) / sd, (qv[j].z * rq) / sd, (qv[j].w * rq) / sd};
                kv[j] = f4v{kv[j].x * rk, kv[j].y * rk, kv[j].z * rk, kv[j].w * rk};
                if (r < n) {
                    const size_t off = size_t(t0 + r) * vh * kD + size_t(h) * kD + i;
                    *reinterpret_cast<f4v*>(a.p[1] + off) = qv[j];
                    *reinterpret_cast<f4v*>(a.p[2] + off) = kv[j];
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kPrepLoads; ++j) {
            const int e = tid + kPrep * j, r = e >> 5, i = (e & 31) * 4;
            *reinterpret_cast<f4v*>(&ks[r][i]) = kv[j];
            *reinterpret_cast<f4v*>(&qs[r][i]) = qv[j];
        }
    }
    if (tid < kC) {  // wave 0: gates and the inclusive prefix of g
        float g = 0.f, b = 0.f;
        if (tid < n) {
            if (gated) {
                g = -expf(galog) * softplusf_(ga + gdt);
                b = sigmoidf_(gb);
            } else {
                g = ga;
                b = gb;
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
    {  // Gram products K K^T and Q K^T on MFMA, the 10 lower 16 x 16 tiles (sj <= ti)
        const int w = tid >> 6, l = tid & 63, lc = l & 15, q = l >> 4;
        for (int e = tid; e < 6 * 256; e += kPrep) {  // the upper tiles are zero
            const int tile = e >> 8, ti = tile < 3 ? 0 : tile < 5 ? 1 : 2, sj = tile < 3 ? tile + 1 : tile < 5 ? tile - 1 : 3;
            const int t = 16 * ti + ((e >> 4) & 15), s2 = 16 * sj + (e & 15);
            lm[t][s2] = 0.f;
        }
        // the 20 products (tile j of the list (ti, sj) = (0,0) (1,0) (1,1) (2,0) ... (3,3), K K^T
        // or Q K^T) dealt to the 8 waves: product w + 8 k
        for (int pr = w; pr < 20; pr += kPrep / 64) {
            const int j = pr >> 1, qk = pr & 1;
            const int ti = j < 1 ? 0 : j < 3 ? 1 : j < 6 ? 2 : 3, sj = j - ti * (ti + 1) / 2;
            // MFMA step 4 m + e, lane (lc, q) takes k = 32 q + 4 m + e: a lane's operands of a
            // tile are 8 contiguous float4 per matrix, read before the 32 MFMAs
            float (*as)[kD + 4] = qk ? qs : ks;
            // two independent accumulator chains (k below and above 64 within each lane group's
            // 32), added at the end
            f4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
            f4v xa[8], xb[8];
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                xa[m] = *reinterpret_cast<const f4v*>(&as[16 * ti + lc][32 * q + 4 * m]);
                xb[m] = *reinterpret_cast<const f4v*>(&ks[16 * sj + lc][32 * q + 4 * m]);
            }
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[m][e], xb[m][e], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[m + 4][e], xb[m + 4][e], acc1, 0, 0, 0);
                }
            const f4v acc = acc0 + acc1;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * ti + 4 * q + r, s2 = 16 * sj + lc;
                const float e = s2 <= t ? expf(float(gd[t] - gd[s2])) : 0.f;
                if (qk)
                    lm[t][s2] = e * acc[r];
                else
                    am[s2][t] = s2 < t ? bs[t] * e * acc[r] : 0.f;
            }
        }
    }
    __syncthreads();
    // e^G Q, (e^{G_63-G} K)^T and L into the record, one float4 of the
    // destination per thread step (contiguous stores)
    for (int d = tid; d < kC * kD / 4; d += kPrep) {
        const int l = d & 63, lr = l & 15, q = l >> 4;
        {  // e^G Q: 4 tiles of 16 rows, K = 128 (8 float4 per lane)
            const int tile = d >> 9, m = (d >> 6) & 7, t = tile * 16 + lr, k = 16 * m + q;
            rec4[kQ / 4 + d] = f4v{qs[t][k], qs[t][k + 4], qs[t][k + 8], qs[t][k + 12]} * eg[t];
        }
        {  // (e^{G_63-G} K)^T: 8 tiles of 16 key dims, K = 64 tokens (4 float4 per lane)
            const int tile = d >> 8, m = (d >> 6) & 3, i = tile * 16 + lr, t = 16 * m + q;
            rec4[kK / 4 + d] = f4v{el[t] * ks[t][i], el[t + 4] * ks[t + 4][i], el[t + 8] * ks[t + 8][i],
                                   el[t + 12] * ks[t + 12][i]};
        }
        if (d < kC * kC / 4) {  // L: 4 tiles of 16 tokens, K = 64 tokens
            const int tile = d >> 8, m = (d >> 6) & 3, t = tile * 16 + lr, k = 16 * m + q;
            rec4[kL / 4 + d] = f4v{lm[t][k], lm[t][k + 4], lm[t][k + 8], lm[t][k + 12]};
        }
    }
    if (tid >= kPrep - 64) {  // the last wave: lane (i, j) = column j of the inverse of diagonal block i,
                              // by forward substitution (y_t = [t == j] - A_t0 y_0 - ..., in that order)
        const int i = (tid & 63) >> 4, j = tid & 15, o = 16 * i;
        float y[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) y[t] = t == j ? 1.f : 0.f;
#pragma unroll
        for (int s2 = 0; s2 < 15; ++s2)
#pragma unroll
            for (int t = s2 + 1; t < 16; ++t) y[t] = fmaf(-am[o + s2][o + t], y[s2], y[t]);
#pragma unroll
        for (int t = 0; t < 16; ++t) li[i][t][j] = y[t];
    }
    __syncthreads();
    {  // right-hand sides: beta e^G K in ks, beta V in qs
#pragma unroll
        for (int j = 0; j < kPrepLoads; ++j) {
            const int e = tid + kPrep * j, t = e >> 5, i = (e & 31) * 4;
            f4v* kr = reinterpret_cast<f4v*>(&ks[t][i]);
            *kr = *kr * (bs[t] * eg[t]);
            *reinterpret_cast<f4v*>(&qs[t][i]) = vv[j] * bs[t];
        }
    }
    __syncthreads();
    {  // (I + A) X = B by blocks of 16 rows on MFMA, B = [beta e^G K | beta V] (256 columns, in
       // ks | qs). Block row i: X_i = ((I + A)_ii)^-1 (B_i - A_{i,<i} X_{<i}): the first
       // product over the solved rows (k = 4 step + lane / 16), the second over the 16 rows of
       // the block with k = 4 (lane / 16) + step, so B_i - A X sits in the accumulator
       // registers that operand needs (no data movement). Wave w owns the 16-column tiles
       // 2 w and 2 w + 1 in every block row, so the solve needs no block barrier (a wave's
       // LDS operations complete in order). The solution replaces B in LDS.
        const int w = tid >> 6, l = tid & 63, lc = l & 15, q = l >> 4;
        constexpr int RS = kD + 4;  // row stride of ks / qs
#pragma unroll
        for (int i = 0; i < kC / 16; ++i) {
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const int tile = 2 * w + ct;  // 16-column tile of the 256 combined columns
                float* base = tile < kD / 16 ? &ks[0][16 * tile] : &qs[0][16 * tile - kD];
                f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 4 * i; ++st) {
                    const int k = 4 * st + q;  // A[16 i + lc][k] = am[k][16 i + lc]
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(am[k][16 * i + lc], base[k * RS + lc], acc, 0, 0, 0);
                }
                f4v b;  // B_i - A X: row 16 i + 4 q + r, column lc
#pragma unroll
                for (int r = 0; r < 4; ++r) b[r] = base[(16 * i + 4 * q + r) * RS + lc] - acc[r];
                const f4v inv = *reinterpret_cast<const f4v*>(&li[i][lc][4 * q]);  // row lc, k = 4 q + st
                f4v x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 4; ++st) x = __builtin_amdgcn_mfma_f32_16x16x4f32(inv[st], b[st], x, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) base[(16 * i + 4 * q + r) * RS + lc] = x[r];
            }
        }
    }
    __syncthreads();
    for (int d = tid; d < kC * kD / 4; d += kPrep) {
        const int l = d & 63, lr = l & 15, q = l >> 4;
        {  // -W, as e^G Q
            const int tile = d >> 9, m = (d >> 6) & 7, t = tile * 16 + lr, k = 16 * m + q;
            rec4[kW / 4 + d] = -f4v{ks[t][k], ks[t][k + 4], ks[t][k + 8], ks[t][k + 12]};
        }
        {  // U in accumulator order
            const int js = (d >> 6) & (kSlices - 1), tile = d >> 9, t = tile * 16 + 4 * q, col = js * 16 + lr;
            rec4[kU / 4 + d] = f4v{qs[t][col], qs[t + 1][col], qs[t + 2][col], qs[t + 3][col]};
        }
    }
    if (tid == 0) rec[kG] = eg[kC - 1];
}

__global__ __launch_bounds__(kPrep) void rule_chunk_prep_kernel(Params a, int gated, int qkn, int c0, float* scratch) {
    __shared__ PrepLds P;
    prep_task(a, gated, qkn, c0, scratch, int(blockIdx.x), int(blockIdx.y), P);
}

__device__ __forceinline__ f4v mfma16(float x, float y, f4v acc) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(x, y, acc, 0, 0, 0);
}

// One block per (head, 16-column slice of S), 4 waves. Wave w: rows 16w..16w+15
// of D and of O (phase 1: D = U - W S0 and O = e^G Q S0, sharing every S0
// read), then O += L D over the tokens up to its rows and S rows of tiles w
// and w + 4 (phase 2: one D read feeds all three products).
// S and D live in LDS in B-operand order: entry [l][s] is row 4 s + l / 16,
// column l % 16, the value lane l feeds the MFMA step s (k = 4 s + l / 16)
// of a product over them, so each lane takes all of its operands in a few
// 16-byte reads and one wait (rows padded to 36 / 20 floats: the 16-byte
// reads of 8 consecutive lanes hit distinct banks).
// Operand loads run a phase ahead: chunk c + 1's -W and e^G Q float4 m are
// issued as soon as phase 1 of chunk c has consumed chunk c's (so the loads
// go out while the MFMAs run), its L and K^T likewise in phase 2; the
// barriers wait for LDS only, so those loads stay in flight across them
// (__syncthreads() would also wait for every outstanding load).
// Blocks are dealt to the 8 XCDs round-robin by index; the index is remapped
// so that the 8 slices of a head run on one XCD: every slice reads the whole
// chunk record, and this way 7 of the 8 reads hit that XCD's L2 instead of
// the memory-side cache or HBM.
constexpr int kXcds = 8;
constexpr int kSRow = 36, kDRow = 20;
typedef __amdgpu_buffer_rsrc_t Rs;
__device__ void buffer_store_f32(float v, Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.store.f32");
// Block barrier for LDS traffic only: the block's LDS writes done
// (lgkmcnt(0)), then s_barrier; outstanding global loads and stores are not
// waited for.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt not waited
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ const float* scan_rec(const float* __restrict__ scratch, int c, int vh, int h) {
    return scratch + (size_t(c) * vh + h) * kRec;
}
// Phase-1 operands of a chunk: -W and e^G Q rows of tile w, U of the slice.
__device__ __forceinline__ void scan_load1(const float* rec, int w, int js, int l, f4v (&wv)[8], f4v (&qv)[8], f4v& uv) {
    const f4v* W = reinterpret_cast<const f4v*>(rec + kW) + w * 512 + l;
    const f4v* Q = reinterpret_cast<const f4v*>(rec + kQ) + w * 512 + l;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        wv[m] = W[m * 64];
        qv[m] = Q[m * 64];
    }
    uv = reinterpret_cast<const f4v*>(rec + kU)[(w * kSlices + js) * 64 + l];
}
// Phase-2 operands: L rows of tile w, K^T rows of tiles w and w + 4.
__device__ __forceinline__ void scan_load2(const float* rec, int w, int l, f4v (&lv)[4], f4v (&k0)[4], f4v (&k1)[4]) {
    const f4v* Lp = reinterpret_cast<const f4v*>(rec + kL) + w * 256 + l;
    const f4v* Kp = reinterpret_cast<const f4v*>(rec + kK) + l;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        lv[m] = Lp[m * 64];
        k0[m] = Kp[w * 256 + m * 64];
        k1[m] = Kp[(w + 4) * 256 + m * 64];
    }
}
struct ScanLds {
    alignas(16) float sl[64][kSRow];
    alignas(16) float dl[64][kDRow];
};
// Block b of nb scan blocks -> its (head, slice) index: the 8 slices of a
// head on one XCD.
__device__ __forceinline__ int scan_index(int b, int nb) {
    return nb % kXcds == 0 ? (b % kXcds) * (nb / kXcds) + b / kXcds : b;
}
// The scan of chunks [c0, c0 + chunks) by the (head, slice) of index i over
// the records in `scratch`. With ALL false the block is larger than 256
// threads: the threads past 256 only take part in the barriers.
template <bool ALL>
__device__ __forceinline__ void scan_group(const Params& a, int c0, int chunks, const float* __restrict__ scratch,
                                           int i, ScanLds& S) {
    auto& sl = S.sl;
    auto& dl = S.dl;
    const bool active = ALL || threadIdx.x < 256;
    const int h = i / kSlices, js = i % kSlices;
    const int tid = threadIdx.x, w = (tid >> 6) & 3, l = tid & 63, lc = l & 15, q = l >> 4;
    const int vh = a.n[3], tokens = a.n[4] > 0 ? a.n[4] : 1;
    float* state = a.p[4] + size_t(h) * kD * kD + js * kSlice;
    // the output as a buffer of exactly tokens x vh x kD floats (its size is
    // checked below 2^31 bytes on the host): stores past it are dropped, so
    // the ragged last chunk needs no per-lane branch around its stores
    const Rs out_rs = __builtin_amdgcn_make_buffer_rsrc(a.p[0], 0, tokens * vh * kD * 4, 0x00020000);
    f4v wv[8], qv[8], uv, lv[4], k0[4], k1[4];
    if (active) {
        for (int e = tid; e < kD * kSlice; e += 256) {  // S row k, column j -> [16 (k % 4) + j][k / 4]
            const int k = e / kSlice, j = e % kSlice;
            sl[16 * (k & 3) + j][k >> 2] = state[size_t(k) * kD + j];
        }
        scan_load1(scan_rec(scratch, 0, vh, h), w, js, l, wv, qv, uv);
        scan_load2(scan_rec(scratch, 0, vh, h), w, l, lv, k0, k1);
    }
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
        const int t0 = (c0 + c) * kC;
        const int cn = c + 1 < chunks ? c + 1 : c;  // the last chunk reloads itself
        const float decay = scan_rec(scratch, c, vh, h)[kG];
        const float* recn = scan_rec(scratch, cn, vh, h);
        f4v oacc = {0.f, 0.f, 0.f, 0.f};
        if (active) {
            f4v sb[8];  // S in B-operand order: step s = 4 m + e is sb[m][e]
#pragma unroll
            for (int m = 0; m < 8; ++m) sb[m] = *reinterpret_cast<const f4v*>(&sl[l][4 * m]);
            f4v dacc = uv;
#pragma unroll
            for (int m = 0; m < 8; ++m) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dacc = mfma16(wv[m][e], sb[m][e], dacc);
                    oacc = mfma16(qv[m][e], sb[m][e], oacc);
                }
                // float4 m is consumed: chunk cn's goes out while the MFMAs run
                wv[m] = reinterpret_cast<const f4v*>(recn + kW)[w * 512 + m * 64 + l];
                qv[m] = reinterpret_cast<const f4v*>(recn + kQ)[w * 512 + m * 64 + l];
            }
            uv = reinterpret_cast<const f4v*>(recn + kU)[(w * kSlices + js) * 64 + l];
#pragma unroll
            for (int r = 0; r < 4; ++r) dl[16 * r + lc][4 * w + q] = dacc[r];  // D row 16 w + 4 q + r
        }
        lds_barrier();
        if (active) {
            f4v s0, s1;
#pragma unroll
            for (int r = 0; r < 4; ++r) {  // S rows 16 w + 4 q + r and 16 (w + 4) + 4 q + r
                s0[r] = decay * sl[16 * r + lc][4 * w + q];
                s1[r] = decay * sl[16 * r + lc][4 * w + 16 + q];
            }
            f4v db[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) db[m] = *reinterpret_cast<const f4v*>(&dl[l][4 * m]);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (m <= w) oacc = mfma16(lv[m][e], db[m][e], oacc);  // L is zero past the tile's last token
                    s0 = mfma16(k0[m][e], db[m][e], s0);
                    s1 = mfma16(k1[m][e], db[m][e], s1);
                }
                const f4v* Kp = reinterpret_cast<const f4v*>(recn + kK) + l;
                lv[m] = reinterpret_cast<const f4v*>(recn + kL)[w * 256 + m * 64 + l];
                k0[m] = Kp[w * 256 + m * 64];
                k1[m] = Kp[(w + 4) * 256 + m * 64];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + 16 * w + 4 * q + r;  // rows t >= tokens fall outside out_rs: dropped
                buffer_store_f32(oacc[r], out_rs, unsigned(((t * vh + h) * kD + js * kSlice + lc) * 4), 0, 0);
                sl[16 * r + lc][4 * w + q] = s0[r];
                sl[16 * r + lc][4 * w + 16 + q] = s1[r];
            }
        }
        lds_barrier();
    }
    __syncthreads();
    if (active)
        for (int e = tid; e < kD * kSlice; e += 256) {
            const int k = e / kSlice, j = e % kSlice;
            state[size_t(k) * kD + j] = sl[16 * (k & 3) + j][k >> 2];
        }
}

__global__ __launch_bounds__(256) void rule_chunk_scan_kernel(Params a, int c0, int chunks,
                                                              const float* __restrict__ scratch) {
    __shared__ ScanLds S;
    scan_group<true>(a, c0, chunks, scratch, scan_index(int(blockIdx.x), int(gridDim.x)), S);
}

// One launch, two jobs on separate CUs: blocks [0, nscan) scan the chunks
// [sc0, sc0 + schunks) from the records in `srec` (as rule_chunk_scan_kernel,
// on 4 of their 8 waves); the others make the records of the next group's
// chunks [pc0, pc0 + pchunks) into `prec`, the (chunk, head) tasks dealt
// round-robin. The two record buffers are disjoint and neither job waits for
// the other. Their LDS together (~122 KiB) leaves room for one block per CU,
// so on an idle device the blocks take one CU each and the prep work never
// shares a CU with the latency-bound scan.
__global__ __launch_bounds__(kPrep) void rule_chunk_scan_prep_kernel(Params a, int gated, int qkn, int nscan, int sc0,
                                                                     int schunks, const float* __restrict__ srec,
                                                                     int pc0, int pchunks, float* prec) {
    __shared__ ScanLds S;
    __shared__ PrepLds P;
    const int b = int(blockIdx.x), vh = a.n[3];
    if (b < nscan) {
        scan_group<false>(a, sc0, schunks, srec, scan_index(b, nscan), S);
        return;
    }
    const int nprep = int(gridDim.x) - nscan;
    for (int task = b - nscan; task < pchunks * vh; task += nprep) {
        if (task != b - nscan) __syncthreads();  // every thread past the previous task's LDS reads
        prep_task(a, gated, qkn, pc0, prec, task / vh, task % vh, P);
    }
}

}  // namespace

bool delta_rule_chunked_ok(const Params& a, int count) {
    const int tokens = a.n[4] > 0 ? a.n[4] : 1;
    const uintptr_t vec = reinterpret_cast<uintptr_t>(a.p[1]) | reinterpret_cast<uintptr_t>(a.p[2]) |
                          reinterpret_cast<uintptr_t>(a.p[3]);  // float4 loads of q, k, v rows
    return a.n[0] == kD && a.n[1] == kD && a.n[3] >= 1 && count == a.n[3] * kD && a.n[6] <= 0 &&
           tokens >= kChunkMinTokens && vec % 16 == 0 && a.n[5] % 4 == 0 && a.n[2] >= 0 &&
           int64_t(tokens) * a.n[3] * kD * 4 < (int64_t(1) << 31);  // the scan's output buffer resource
}

// Chunks per group. Up to kOneGroup chunks: one group (the prep on every CU,
// then the scan). Beyond: groups of about kGroupTarget chunks, equal in size,
// the scan of group g and the prep of group g + 1 in one launch; at that size
// the prep of a group on the CUs the scan leaves free takes about as long as
// its scan (measured at 10,240 tokens of the 0.8B shape: 633 -> 608 us per
// layer for prep + scan; 8-chunk groups 668 us, the launches' fixed cost; at
// 2644 tokens three overlapped groups measured no faster than one).
constexpr int kOneGroup = 64, kGroupTarget = 16;
int group_chunks(int chunks) {
    if (chunks <= kOneGroup) return chunks;
    const int groups = (chunks + kGroupTarget - 1) / kGroupTarget;
    return (chunks + groups - 1) / groups;
}

size_t delta_rule_chunked_scratch(const Params& a) {
    const int tokens = a.n[4] > 0 ? a.n[4] : 1;
    const int chunks = int(ceil_div(tokens, kC)), g = group_chunks(chunks);
    return size_t(chunks > g ? 2 : 1) * size_t(g) * size_t(a.n[3]) * kRec;
}

int run_delta_rule_chunked(hipStream_t s, bool gated, const Params& a, float* scratch, size_t len, bool qkn) {
    if (len < delta_rule_chunked_scratch(a)) return int(hipErrorInvalidValue);
    const int tokens = a.n[4] > 0 ? a.n[4] : 1, vh = a.n[3];
    if (qkn && (a.n[2] < 1 || vh % a.n[2] != 0)) return int(hipErrorInvalidValue);
    const int chunks = int(ceil_div(tokens, kC)), g = group_chunks(chunks);
    float* buf[2] = {scratch, scratch + size_t(g) * size_t(vh) * kRec};
    const int nscan = vh * kSlices, nprep = nscan < 256 - 64 ? 256 - nscan : 64;
    hipLaunchKernelGGL(rule_chunk_prep_kernel, dim3(unsigned(g), unsigned(vh)), dim3(kPrep), 0, s, a, gated ? 1 : 0,
                       qkn ? 1 : 0, 0, buf[0]);
    if (hipError_t e = hipGetLastError()) return int(e);
    for (int c0 = 0, k = 0; c0 < chunks; c0 += g, ++k) {
        const int n = chunks - c0 < g ? chunks - c0 : g, c1 = c0 + n;
        if (c1 < chunks) {  // this group's scan beside the next group's prep
            const int n1 = chunks - c1 < g ? chunks - c1 : g;
            hipLaunchKernelGGL(rule_chunk_scan_prep_kernel, dim3(unsigned(nscan + nprep)), dim3(kPrep), 0, s, a,
                               gated ? 1 : 0, qkn ? 1 : 0, nscan, c0, n, static_cast<const float*>(buf[k & 1]), c1, n1,
                               buf[(k + 1) & 1]);
        } else {
            hipLaunchKernelGGL(rule_chunk_scan_kernel, dim3(unsigned(nscan)), dim3(256), 0, s, a, c0, n,
                               static_cast<const float*>(buf[k & 1]));
        }
        if (hipError_t e = hipGetLastError()) return int(e);
    }
    return 0;
}

}  // namespace qr
