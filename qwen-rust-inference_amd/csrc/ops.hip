// qr_run ops on gfx950: elementwise ops, the RMSNorm family, DeltaNet conv /
// Q-K normalisation / gates / recurrent rule, attention Q/K preparation with
// partial RoPE, embedding rows and the two-pass argmax.
//
// Each op computes what the reference's op body computes
// (native/rocm/reference.h:117-232, slot meanings there); the decomposition is
// this file's own: a wave or block per group for reductions, P lanes per
// DeltaNet value column with the column's state in VGPRs.
#include <mutex>

#include "common.h"

namespace qr {
namespace {

// ---------------------------------------------------------------- elementwise
// Add (2), SiluProduct (3), DeltaGates (6), EmbedBf16 (11), EmbedBf16Picked (17).
__global__ __launch_bounds__(256) void elementwise_kernel(int op, int count, Params a) {
    for (long t = blockIdx.x * long(blockDim.x) + threadIdx.x; t < count; t += long(gridDim.x) * blockDim.x) {
        switch (op) {
        case QR_ADD: a.p[0][t] = a.p[1][t] + a.p[2][t]; break;
        case QR_SILU_PRODUCT: a.p[0][t] = siluf_(a.p[1][t]) * a.p[2][t]; break;
        case QR_DELTA_GATES: {  // reference.h:144-148
            int head = a.n[0] > 0 ? int(t % a.n[0]) : int(t);
            a.p[0][t] = -expf(a.p[4][head]) * softplusf_(a.p[1][t] + a.p[3][head]);
            a.p[5][t] = sigmoidf_(a.p[2][t]);
            break;
        }
        case QR_EMBED_BF16: {  // reference.h:213-216
            const uint16_t* m = reinterpret_cast<const uint16_t*>(a.p[1]);
            a.p[0][t] = __uint_as_float(uint32_t(m[size_t(a.n[0]) * size_t(a.n[1]) + size_t(t)]) << 16);
            break;
        }
        case QR_EMBED_BF16_PICKED: {  // reference.h:217-221
            const uint16_t* m = reinterpret_cast<const uint16_t*>(a.p[1]);
            size_t h = size_t(a.n[1]), r = size_t(t) / h;
            size_t row = size_t(a.p[2][2 * r]);
            a.p[0][t] = __uint_as_float(uint32_t(m[row * h + size_t(t) % h]) << 16);
            break;
        }
        }
    }
}

// Add and SiluProduct four elements per thread (count % 4 == 0, operands
// 16-byte aligned): one 16-byte load per operand.
__global__ __launch_bounds__(256) void elementwise4_kernel(int op, int count4, Params a) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    for (long t = blockIdx.x * long(blockDim.x) + threadIdx.x; t < count4; t += long(gridDim.x) * blockDim.x) {
        const f4 x = reinterpret_cast<const f4*>(a.p[1])[t], y = reinterpret_cast<const f4*>(a.p[2])[t];
        f4 r;
        if (op == QR_ADD) {
            r = x + y;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = siluf_(x[e]) * y[e];
        }
        reinterpret_cast<f4*>(a.p[0])[t] = r;
    }
}

// ---------------------------------------------------------------- RMSNorm family
// RmsNorm (1), AddRmsNorm (12), RmsNormGate (13): reference.h:120-126,194-207.
// One wave per group when d <= 256, else one block per group.
template <bool WAVE>
__global__ __launch_bounds__(256) void rms_family_kernel(int op, int groups, Params a) {
    __shared__ float red[16];
    const int d = a.n[0];
    const int g = WAVE ? blockIdx.x * 4 + int(threadIdx.x >> 6) : blockIdx.x;
    const int t0 = WAVE ? int(threadIdx.x & 63) : int(threadIdx.x);
    const int step = WAVE ? 64 : int(blockDim.x);
    if (WAVE && g >= groups) return;  // whole waves only: no block barrier in the wave form
    const size_t off = size_t(g) * d;
    const float eps = a.f[0], offset = a.f[1];
    float ss = 0.f;
    if (op == QR_ADD_RMS_NORM) {
        for (int i = t0; i < d; i += step) {
            float s = a.p[1][off + i] + a.p[2][off + i];
            a.p[0][off + i] = s;
            ss += s * s;
        }
    } else {
        for (int i = t0; i < d; i += step) {
            float v = a.p[1][off + i];
            ss += v * v;
        }
    }
    ss = WAVE ? wave_sum(ss) : block_sum(ss, red);
    const float r = 1.f / sqrtf(ss / float(d) + eps);
    for (int i = t0; i < d; i += step) {
        switch (op) {
        case QR_RMS_NORM: a.p[0][off + i] = (a.p[1][off + i] * r) * (a.p[2][i] + offset); break;
        case QR_ADD_RMS_NORM: a.p[3][off + i] = (a.p[0][off + i] * r) * (a.p[4][i] + offset); break;
        case QR_RMS_NORM_GATE:
            a.p[0][off + i] = siluf_(a.p[3][off + i]) * ((a.p[1][off + i] * r) * (a.p[2][i] + offset));
            break;
        }
    }
}

// The same ops with one wave per group and the group in registers when
// d = 64 PER: lane l holds elements V (l + 64 j) .. + V - 1 (V = min(PER, 4),
// j < PER / V), so every load and store of a wave is one contiguous run and
// each input is read once (the block form above reads a group twice and
// waits on two block barriers).
// planes (may be null): the output also as the P3 planes a prepared
// projection takes (common.h), the output read as rows of `width` values (a
// multiple of d and of 32: consecutive groups form a row); the V consecutive
// values of a lane are V consecutive BF16 of each plane. A plane's 128-byte
// lines hold 8 rows: with planes, the blocks are renumbered so that each XCD
// (blocks are dealt to the 8 XCDs round-robin) takes one contiguous range of
// rows, and the rows that share a line are written through one L2.
__device__ __forceinline__ int xcd_contiguous(int b, int nb) {
    const int x = b % 8, per = nb / 8, extra = nb % 8;
    return x * per + (x < extra ? x : extra) + b / 8;
}
template <int PER>
__global__ __launch_bounds__(256) void rms_rows_kernel(int op, int groups, Params a, __bf16* planes, int width) {
    constexpr int V = PER >= 4 ? 4 : PER, NV = PER / V;
    typedef float fv __attribute__((ext_vector_type(V)));
    typedef __bf16 hv __attribute__((ext_vector_type(V)));
    const int b = planes ? xcd_contiguous(int(blockIdx.x), int(gridDim.x)) : int(blockIdx.x);
    const int g = b * 4 + int(threadIdx.x >> 6);
    if (g >= groups) return;  // whole waves only: no block barrier
    const int lane = int(threadIdx.x & 63), d = 64 * PER;
    const size_t off = size_t(g) * d;
    const float eps = a.f[0], offset = a.f[1];
    // Every load of the row (input, the added input, norm weights, gate) is
    // issued before the first store: with the stores in between, the compiler
    // (which cannot rule out aliasing) waited for each 16-byte piece in turn.
    const float* w = op == QR_ADD_RMS_NORM ? a.p[4] : a.p[2];
    float* out = op == QR_ADD_RMS_NORM ? a.p[3] : a.p[0];
    fv x[NV], x2[NV], wv[NV], z[NV];
    const bool add = op == QR_ADD_RMS_NORM, gate = op == QR_RMS_NORM_GATE;
    const float* x2p = add ? a.p[2] : a.p[1];  // the added input, else a second read of x (not used)
    const float* zp = gate ? a.p[3] + off : w;  // the gate's z, else the weights again (not used)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const size_t i = off + size_t(V) * (lane + 64 * j);
        const int c = V * (lane + 64 * j);
        x[j] = *reinterpret_cast<const fv*>(a.p[1] + i);
        x2[j] = *reinterpret_cast<const fv*>(x2p + i);
        wv[j] = *reinterpret_cast<const fv*>(w + c);
        z[j] = *reinterpret_cast<const fv*>(zp + c);
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (add) {
            x[j] += x2[j];
            *reinterpret_cast<fv*>(a.p[0] + off + size_t(V) * (lane + 64 * j)) = x[j];
        }
#pragma unroll
        for (int e = 0; e < V; ++e) ss += x[j][e] * x[j][e];
    }
    ss = wave_sum(ss);
    const float r = 1.f / sqrtf(ss / float(d) + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = V * (lane + 64 * j);
        fv y;
#pragma unroll
        for (int e = 0; e < V; ++e) y[e] = (x[j][e] * r) * (wv[j][e] + offset);
        if (gate) {
#pragma unroll
            for (int e = 0; e < V; ++e) y[e] = siluf_(z[j][e]) * y[e];
        }
        *reinterpret_cast<fv*>(out + off + c) = y;
        if (planes) {
            hv h[3];
#pragma unroll
            for (int e = 0; e < V; ++e) {
                h[0][e] = __bf16(y[e]);
                const float r1 = y[e] - float(h[0][e]);
                h[1][e] = __bf16(r1);
                h[2][e] = __bf16(r1 - float(h[1][e]));
            }
            const unsigned pe = unsigned(off) + unsigned(c), pr = pe / unsigned(width);  // element, plane row
            const int k = int(pe - pr * unsigned(width));
#pragma unroll
            for (int q = 0; q < 3; ++q) *reinterpret_cast<hv*>(planes + p3_index(int(pr), k, q, width / 16)) = h[q];
        }
    }
}

// RmsNormGate with the output's P3 planes for groups of 128 (the DeltaNet
// gated norm before out_proj): one block per (32 rows of the planes, one
// group column h of the width); wave w normalizes rows 8 w .. 8 w + 7 of the
// tile exactly as rms_rows_kernel<2> does (lane l: elements 2 l, 2 l + 1; the
// same sums and products), stores the fp32 output, and stages it in LDS; then
// each wave writes whole 1 KiB plane fragments (rows of the tile x 16 k) for
// two of the group's 8 k tiles. rms_rows_kernel writes a row's planes 4 bytes
// per lane, one cache line each. Rows past `rows` get zero planes.
__global__ __launch_bounds__(256) void rms_gate_planes_kernel(int rows, Params a, __bf16* planes, int width) {
    constexpr int D = 128, KT = D / 16;
    typedef float f2v __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
    __shared__ float ys[32][D + 4];
    const int rt = int(blockIdx.x), h = int(blockIdx.y), hc = width / D;
    const int w = int(threadIdx.x >> 6), lane = int(threadIdx.x & 63);
    const float eps = a.f[0], offset = a.f[1];
    const f2v wv = *reinterpret_cast<const f2v*>(a.p[2] + 2 * lane);
    for (int i = 0; i < 8; ++i) {
        const int rr = 8 * w + i, row = 32 * rt + rr;
        f2v y = {0.f, 0.f};
        if (row < rows) {  // wave-uniform
            const size_t off = (size_t(row) * hc + h) * D + 2 * lane;
            const f2v x = *reinterpret_cast<const f2v*>(a.p[1] + off);
            float ss = 0.f;
            ss += x[0] * x[0];
            ss += x[1] * x[1];
            ss = wave_sum(ss);
            const float r = 1.f / sqrtf(ss / float(D) + eps);
            const f2v z = *reinterpret_cast<const f2v*>(a.p[3] + off);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                y[e] = (x[e] * r) * (wv[e] + offset);
                y[e] = siluf_(z[e]) * y[e];
            }
            *reinterpret_cast<f2v*>(a.p[0] + off) = y;
        }
        ys[rr][2 * lane] = y[0];
        ys[rr][2 * lane + 1] = y[1];
    }
    __syncthreads();
    const int rl = lane & 31, k8 = 8 * (lane >> 5);
    for (int kk = w; kk < KT; kk += 4) {
        bf16x8 hp[3];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = ys[rl][16 * kk + k8 + e];
            const __bf16 h0 = __bf16(v);
            const float r1 = v - float(h0);
            const __bf16 h1 = __bf16(r1);
            hp[0][e] = h0;
            hp[1][e] = h1;
            hp[2][e] = __bf16(r1 - float(h1));
        }
#pragma unroll
        for (int q = 0; q < 3; ++q)
            *reinterpret_cast<bf16x8*>(planes + p3_index(32 * rt + rl, h * D + 16 * kk + k8, q, width / 16)) = hp[q];
    }
}

// ---------------------------------------------------------------- ConvSilu (4)
// reference.h:96-116: one channel per thread, tokens in order through the
// channel's history (oldest -> newest); with n3 = S > 0 the history after
// token r < S is also stored as snapshot r at (r + 1) * n2 * (k - 1).
__global__ __launch_bounds__(256) void conv_silu_kernel(int count, Params a) {
    const int ch = blockIdx.x * blockDim.x + threadIdx.x;
    if (ch >= count) return;
    const int k = a.n[0], tokens = a.n[1] > 0 ? a.n[1] : 1, stride = a.n[2], snaps = a.n[3];
    const float* w = a.p[2] + size_t(ch) * k;
    float* hist = a.p[3] + size_t(ch) * (k - 1);
    float h[16];
    float wk[17];
    for (int i = 0; i < k - 1; ++i) h[i] = hist[i];
    for (int i = 0; i < k; ++i) wk[i] = w[i];
    for (int r = 0; r < tokens; ++r) {
        const float xv = a.p[1][size_t(r) * stride + ch];
        float sum = 0.f;
        for (int i = 0; i < k - 1; ++i) sum += h[i] * wk[i];
        sum += xv * wk[k - 1];
        for (int i = 0; i + 1 < k - 1; ++i) h[i] = h[i + 1];
        if (k > 1) h[k - 2] = xv;
        a.p[0][size_t(r) * stride + ch] = siluf_(sum);
        if (r < snaps)
            for (int i = 0; i < k - 1; ++i) hist[size_t(r + 1) * size_t(stride) * size_t(k - 1) + i] = h[i];
    }
    for (int i = 0; i < k - 1; ++i) hist[i] = h[i];
}

// Prefill form of ConvSilu: one thread per (token, channel); the input at
// relative position j < 0 is history[k - 1 + j]. Same sums as above
// (history terms oldest first, then the new input). Snapshot slot r + 1 gets
// the history after token r (r < snaps). The live history is rewritten by
// conv_history_kernel afterwards, once every token has read it.
__global__ __launch_bounds__(256) void conv_silu_tokens_kernel(int count, Params a) {
    const int ch = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
    if (ch >= count) return;
    const int k = a.n[0], stride = a.n[2], snaps = a.n[3];
    const float* w = a.p[2] + size_t(ch) * k;
    const float* hist = a.p[3] + size_t(ch) * (k - 1);
    auto input = [&](int j) { return j >= 0 ? a.p[1][size_t(j) * stride + ch] : hist[k - 1 + j]; };
    float sum = 0.f;
    for (int i = 0; i < k - 1; ++i) sum += input(r - (k - 1) + i) * w[i];
    sum += input(r) * w[k - 1];
    a.p[0][size_t(r) * stride + ch] = siluf_(sum);
    if (r < snaps)
        for (int i = 0; i < k - 1; ++i)
            a.p[3][size_t(r + 1) * size_t(stride) * size_t(k - 1) + size_t(ch) * (k - 1) + i] = input(r - (k - 2) + i);
}
// The same for kernel size K, CT tokens per thread: the window of the CT
// tokens' inputs (plus the K - 1 before them) is loaded once, all loads in
// flight together, and slid in registers.
template <int K, int CT>
__global__ __launch_bounds__(256) void conv_silu_window_kernel(int count, Params a) {
    const int ch = blockIdx.x * blockDim.x + threadIdx.x, r0 = int(blockIdx.y) * CT;
    if (ch >= count) return;
    const int tokens = a.n[1], stride = a.n[2], snaps = a.n[3];
    float w[K], win[CT + K - 1];
#pragma unroll
    for (int i = 0; i < K; ++i) w[i] = a.p[2][size_t(ch) * K + i];
    const float* hist = a.p[3] + size_t(ch) * (K - 1);
#pragma unroll
    for (int i = 0; i < CT + K - 1; ++i) {
        const int j = r0 - (K - 1) + i;
        win[i] = j < 0 ? hist[K - 1 + j] : j < tokens ? a.p[1][size_t(j) * stride + ch] : 0.f;
    }
#pragma unroll
    for (int c = 0; c < CT; ++c) {
        const int r = r0 + c;
        if (r >= tokens) break;
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < K - 1; ++i) sum += win[c + i] * w[i];
        sum += win[c + K - 1] * w[K - 1];
        a.p[0][size_t(r) * stride + ch] = siluf_(sum);
        if (r < snaps)
#pragma unroll
            for (int i = 0; i < K - 1; ++i)
                a.p[3][size_t(r + 1) * size_t(stride) * (K - 1) + size_t(ch) * (K - 1) + i] = win[c + 1 + i];
    }
}
__global__ __launch_bounds__(256) void conv_history_kernel(int count, Params a) {
    const int ch = blockIdx.x * blockDim.x + threadIdx.x;
    if (ch >= count) return;
    const int k = a.n[0], tokens = a.n[1], stride = a.n[2];
    float* hist = a.p[3] + size_t(ch) * (k - 1);
    float h[16];
    for (int i = 0; i < k - 1; ++i) {
        const int j = tokens - (k - 1) + i;
        h[i] = j >= 0 ? a.p[1][size_t(j) * stride + ch] : hist[k - 1 + j];
    }
    for (int i = 0; i < k - 1; ++i) hist[i] = h[i];
}

// ---------------------------------------------------------------- DeltaQk (5)
// reference.h:134-143: per (token, value head) the L2-normalised query (then
// / sqrt(d)) and key of its key head. One wave per item.
// DeltaQk for d = 128 with each row in registers: lane l holds elements
// 2 l, 2 l + 1 of q and of k (one 8-byte load each, the row read once).
__global__ __launch_bounds__(256) void delta_qk_pairs_kernel(int count, Params a) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const int t = blockIdx.x * 4 + int(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= count) return;
    constexpr int d = 128;
    const int kh = a.n[0], vh = a.n[1], h = (t % vh) / (vh / kh), kd = kh * d;
    const float* x = a.p[1] + size_t(t / vh) * a.n[3];
    const f2 q = *reinterpret_cast<const f2*>(x + h * d + 2 * lane);
    const f2 k = *reinterpret_cast<const f2*>(x + kd + h * d + 2 * lane);
    const float sq = wave_sum(q.x * q.x + q.y * q.y), sk = wave_sum(k.x * k.x + k.y * k.y);
    const float rq = 1.f / sqrtf(sq + 1e-6f), rk = 1.f / sqrtf(sk + 1e-6f), sd = sqrtf(float(d));
    *reinterpret_cast<f2*>(a.p[0] + size_t(t) * d + 2 * lane) = f2{(q.x * rq) / sd, (q.y * rq) / sd};
    *reinterpret_cast<f2*>(a.p[2] + size_t(t) * d + 2 * lane) = f2{k.x * rk, k.y * rk};
}
__global__ __launch_bounds__(256) void delta_qk_kernel(int count, Params a) {
    const int t = blockIdx.x * 4 + int(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= count) return;
    const int kh = a.n[0], vh = a.n[1], d = a.n[2], h = (t % vh) / (vh / kh), kd = kh * d;
    const float* x = a.p[1] + size_t(t / vh) * a.n[3];
    float sq = 0.f, sk = 0.f;
    for (int i = lane; i < d; i += 64) {
        float q = x[h * d + i], kk = x[kd + h * d + i];
        sq += q * q;
        sk += kk * kk;
    }
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    const float rq = 1.f / sqrtf(sq + 1e-6f), rk = 1.f / sqrtf(sk + 1e-6f), sd = sqrtf(float(d));
    for (int i = lane; i < d; i += 64) {
        a.p[0][size_t(t) * d + i] = (x[h * d + i] * rq) / sd;
        a.p[2][size_t(t) * d + i] = x[kd + h * d + i] * rk;
    }
}

// ---------------------------------------------------------------- DeltaRule (7, 14)
// reference.h:149-170 (and the gate expressions of reference.h:48-60): state
// S[head][key][value]; per token S <- e^g S, m_j = sum_i S_ij k_i,
// delta_j = (v_j - m_j) beta, S_ij += k_i delta_j, o_j = sum_i S_ij q_i.
// Decomposition: P lanes share one value column, each holding KR key rows of
// it in VGPRs (lane = p * (64 / P) + column-in-wave); the column sums are
// reduced over the P lanes with two shuffles. Tokens run in order with the
// state resident; snapshots (n6 = S > 0) store the state after token r < S at
// (r + 1) * vh * kd * vd.
template <int KR, int P, bool GATED>
__global__ __launch_bounds__(256) void delta_rule_kernel(int count, Params a) {
    constexpr int CW = 64 / P;  // columns per wave
    const int lane = threadIdx.x & 63, p = lane / CW, jj = lane % CW;
    const int col = (blockIdx.x * 4 + int(threadIdx.x >> 6)) * CW + jj;
    const bool active = col < count;
    const int kd = a.n[0], vd = a.n[1], kh = a.n[2], vh = a.n[3];
    const int tokens = a.n[4] > 0 ? a.n[4] : 1, stride = a.n[5], snaps = a.n[6];
    const int h = active ? col / vd : 0, j = active ? col % vd : 0;
    float* state = a.p[4] + size_t(h) * kd * vd;
    float s[KR];
#pragma unroll
    for (int ii = 0; ii < KR; ++ii) {
        const int i = p * KR + ii;
        s[ii] = active && i < kd ? state[size_t(i) * vd + j] : 0.f;
    }
    for (int r = 0; r < tokens; ++r) {
        const float* q = a.p[1] + size_t(r) * vh * kd + size_t(h) * kd;
        const float* k = a.p[2] + size_t(r) * vh * kd + size_t(h) * kd;
        float log_decay = 0.f, beta = 0.f, v = 0.f;
        if (active) {
            const int gi = r * vh + h;
            if (GATED) {
                log_decay = -expf(a.p[7][vh + h]) * softplusf_(a.p[5][gi] + a.p[7][h]);
                beta = sigmoidf_(a.p[6][gi]);
            } else {
                log_decay = a.p[5][gi];
                beta = a.p[6][gi];
            }
            v = a.p[3][size_t(r) * stride + 2 * size_t(kh) * kd + size_t(h) * vd + j];
        }
        const float decay = expf(log_decay);
        float kv[KR], qv[KR];
        float m = 0.f;
#pragma unroll
        for (int ii = 0; ii < KR; ++ii) {
            const int i = p * KR + ii;
            kv[ii] = active && i < kd ? k[i] : 0.f;
            qv[ii] = active && i < kd ? q[i] : 0.f;
            s[ii] *= decay;
            m = fmaf(s[ii], kv[ii], m);
        }
#pragma unroll
        for (int o = CW; o < 64; o <<= 1) m += __shfl_xor(m, o, 64);
        const float delta = (v - m) * beta;
        float out = 0.f;
#pragma unroll
        for (int ii = 0; ii < KR; ++ii) {
            s[ii] = fmaf(kv[ii], delta, s[ii]);
            out = fmaf(s[ii], qv[ii], out);
        }
#pragma unroll
        for (int o = CW; o < 64; o <<= 1) out += __shfl_xor(out, o, 64);
        if (active && p == 0) a.p[0][size_t(r) * vh * vd + col] = out;
        if (active && r < snaps) {
            float* snap = state + size_t(r + 1) * vh * kd * vd;
#pragma unroll
            for (int ii = 0; ii < KR; ++ii) {
                const int i = p * KR + ii;
                if (i < kd) snap[size_t(i) * vd + j] = s[ii];
            }
        }
    }
    if (active) {
#pragma unroll
        for (int ii = 0; ii < KR; ++ii) {
            const int i = p * KR + ii;
            if (i < kd) state[size_t(i) * vd + j] = s[ii];
        }
    }
}

// ---------------------------------------------------------------- attention Q / KV
// AttentionQuery (8), AttentionKv (9), AttentionQueryKv (15): reference.h:61-95.
// One block per item; the head vector is normalised into LDS and RoPE'd there.
// `denom[i]` = theta^(2i / rot), computed once on the host with the same libm
// powf the CPU path calls, so the angle pos / denom[i] is the same correctly
// rounded quotient on both sides (a one-ulp powf difference alone moves the
// angle by ~5e-4 rad at position 8190).
__device__ void rope_lds(float* o, int rot, int pos, const float* denom) {
    for (int i = threadIdx.x; i < rot / 2; i += blockDim.x) {
        float angle = float(pos) / denom[i];
        float sn = sinf(angle), cs = cosf(angle);
        float x0 = o[i], x1 = o[i + rot / 2];
        o[i] = x0 * cs - x1 * sn;
        o[i + rot / 2] = x1 * cs + x0 * sn;
    }
}

__device__ void attention_query_item(int t, const Params& a, const float* denom, float* buf, float* red) {
    const int d = a.n[0], rot = a.n[1], pos = a.n[2] + (a.n[3] > 0 ? t / a.n[3] : 0);
    const float* x = a.p[1] + size_t(t) * 2 * d;
    float ss = 0.f;
    for (int i = threadIdx.x; i < d; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    const float r = 1.f / sqrtf(ss / float(d) + a.f[0]);
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        buf[i] = (x[i] * r) * (1.f + a.p[2][i]);
        a.p[3][size_t(t) * d + i] = x[d + i];
    }
    __syncthreads();
    rope_lds(buf, rot, pos, denom);
    __syncthreads();
    for (int i = threadIdx.x; i < d; i += blockDim.x) a.p[0][size_t(t) * d + i] = buf[i];
}

__device__ void attention_kv_item(int t, const Params& a, const float* denom, float* buf, float* red) {
    const int d = a.n[0], rot = a.n[1], kv = a.n[3], pos = a.n[2] + t / kv, hh = t % kv;
    const float* x = a.p[1] + size_t(t) * d;
    float ss = 0.f;
    for (int i = threadIdx.x; i < d; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    const float r = 1.f / sqrtf(ss / float(d) + a.f[0]);
    const size_t dest = (size_t(pos) * kv + hh) * d;
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        buf[i] = (x[i] * r) * (1.f + a.p[2][i]);
        a.p[4][dest + i] = a.p[3][size_t(t) * d + i];
    }
    __syncthreads();
    rope_lds(buf, rot, pos, denom);
    __syncthreads();
    for (int i = threadIdx.x; i < d; i += blockDim.x) a.p[0][dest + i] = buf[i];
}

constexpr int kAttnMaxHeadDim = 1024;

__global__ __launch_bounds__(256) void attention_qkv_kernel(int op, int count, Params a, const float* denom) {
    __shared__ float buf[kAttnMaxHeadDim];
    __shared__ float red[16];
    const int t = blockIdx.x;
    if (op == QR_ATTENTION_QUERY) {
        attention_query_item(t, a, denom, buf, red);
    } else if (op == QR_ATTENTION_KV) {
        attention_kv_item(t, a, denom, buf, red);
    } else {  // AttentionQueryKv: split the items as reference.h:65-74 does
        const int queries = a.n[3] * a.n[5];
        Params part{};
        part.n[0] = a.n[0];
        part.n[1] = a.n[1];
        part.n[2] = a.n[2];
        part.f[0] = a.f[0];
        part.f[1] = a.f[1];
        if (t < queries) {
            part.p[0] = a.p[0];
            part.p[1] = a.p[1];
            part.p[2] = a.p[2];
            part.p[3] = a.p[3];
            part.n[3] = a.n[3];
            attention_query_item(t, part, denom, buf, red);
        } else {
            part.p[0] = a.p[4];
            part.p[1] = a.p[5];
            part.p[2] = a.p[2] + a.n[0];
            part.p[3] = a.p[6];
            part.p[4] = a.p[7];
            part.n[3] = a.n[4];
            attention_kv_item(t - queries, part, denom, buf, red);
        }
    }
    (void)count;
}

// The same items with one wave each (four per 256-thread block) when d = 64
// NJ and rot <= 64: lane l holds elements l + 64 j, the rotary partner of
// element i < rot / 2 (i + rot / 2) sits in lane l + rot / 2 of the same
// register, so no block barrier or LDS round trip is needed (the block form
// spends most of its time on those at d = 256: 102,400 blocks at 10,240
// tokens). The sum of squares is formed exactly as block_sum forms it for a
// 256-thread block (thread 64 w + l accumulates elements 64 w + l + 256 m in m
// order, one butterfly per wave, the wave sums added in order), so the
// results equal the block form's.
template <int NJ>
__device__ __forceinline__ void qkv_item_wave(bool query, int t, const Params& a, const float* denom, int l) {
    constexpr int d = 64 * NJ;
    const int rot = a.n[1], half = rot / 2;
    int pos;
    const float* x;
    float* out;
    size_t dest = 0;
    if (query) {
        pos = a.n[2] + (a.n[3] > 0 ? t / a.n[3] : 0);
        x = a.p[1] + size_t(t) * 2 * d;
        out = a.p[0] + size_t(t) * d;
    } else {
        const int kv = a.n[3];
        pos = a.n[2] + t / kv;
        x = a.p[1] + size_t(t) * d;
        dest = (size_t(pos) * kv + t % kv) * d;
        out = a.p[0] + dest;
    }
    float v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) v[j] = x[l + 64 * j];
    float ss = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        float part = 0.f;
#pragma unroll
        for (int j = w; j < NJ; j += 4) part += v[j] * v[j];
        ss += wave_sum(part);
    }
    const float r = 1.f / sqrtf(ss / float(d) + a.f[0]);
    float y[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int e = l + 64 * j;
        y[j] = (v[j] * r) * (1.f + a.p[2][e]);
        if (query)
            a.p[3][size_t(t) * d + e] = x[d + e];
        else
            a.p[4][dest + e] = a.p[3][size_t(t) * d + e];
    }
    // rope_lds on element pairs (i, i + half), i < half, all in j = 0
    const int partner = l < half ? l + half : l < rot ? l - half : l;
    const float pv = __shfl(y[0], partner, kWave);
    if (l < rot) {
        const int i = l < half ? l : l - half;
        const float angle = float(pos) / denom[i];
        const float sn = sinf(angle), cs = cosf(angle);
        y[0] = l < half ? y[0] * cs - pv * sn : y[0] * cs + pv * sn;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) out[l + 64 * j] = y[j];
}

template <int NJ>
__global__ __launch_bounds__(256) void attention_qkv_wave_kernel(int op, int count, Params a, const float* denom) {
    const int item = int(blockIdx.x) * 4 + int(threadIdx.x >> 6), l = int(threadIdx.x & 63);
    if (item >= count) return;  // whole waves only: no block barrier
    if (op == QR_ATTENTION_QUERY) {
        qkv_item_wave<NJ>(true, item, a, denom, l);
    } else if (op == QR_ATTENTION_KV) {
        qkv_item_wave<NJ>(false, item, a, denom, l);
    } else {  // AttentionQueryKv: the items split as attention_qkv_kernel splits them
        const int queries = a.n[3] * a.n[5];
        Params part{};
        part.n[0] = a.n[0];
        part.n[1] = a.n[1];
        part.n[2] = a.n[2];
        part.f[0] = a.f[0];
        part.f[1] = a.f[1];
        if (item < queries) {
            part.p[0] = a.p[0];
            part.p[1] = a.p[1];
            part.p[2] = a.p[2];
            part.p[3] = a.p[3];
            part.n[3] = a.n[3];
            qkv_item_wave<NJ>(true, item, part, denom, l);
        } else {
            part.p[0] = a.p[4];
            part.p[1] = a.p[5];
            part.p[2] = a.p[2] + a.n[0];
            part.p[3] = a.p[6];
            part.p[4] = a.p[7];
            part.n[3] = a.n[4];
            qkv_item_wave<NJ>(false, item - queries, part, denom, l);
        }
    }
}

// ---------------------------------------------------------------- Argmax (16)
// reference.h:222-230: per row [first index of the maximum over finite values
// (0xffffffff if none), non-finite count]. Pass 1: one block per (slice, row)
// gives (max, index, bad); pass 2: one block per row merges the slices.
constexpr int kArgmaxSlice = 8192;

struct Best {
    float v;
    unsigned i;
    unsigned bad;
};
__device__ __forceinline__ Best better(Best a, Best b) {
    Best r;
    r.bad = a.bad + b.bad;
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) {
        r.v = b.v;
        r.i = b.i;
    } else {
        r.v = a.v;
        r.i = a.i;
    }
    return r;
}
__device__ Best block_best(Best b) {
    __shared__ float sv[16];
    __shared__ unsigned si[16], sb[16];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        Best other{__shfl_xor(b.v, o, 64), unsigned(__shfl_xor(int(b.i), o, 64)),
                   unsigned(__shfl_xor(int(b.bad), o, 64))};
        b = better(b, other);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) {
        sv[wave] = b.v;
        si[wave] = b.i;
        sb[wave] = b.bad;
    }
    __syncthreads();
    Best t{-INFINITY, 0xffffffffu, 0u};
    for (int w = 0; w < waves; ++w) t = better(t, Best{sv[w], si[w], sb[w]});
    return t;
}

__global__ __launch_bounds__(256) void argmax_slices_kernel(Params a, float* parts, int slices) {
    const int n = a.n[0], row = blockIdx.y, slice = blockIdx.x;
    const float* v = a.p[1] + size_t(row) * n;
    const int begin = slice * kArgmaxSlice, end = min(n, begin + kArgmaxSlice);
    Best b{-INFINITY, 0xffffffffu, 0u};
    for (int i = begin + threadIdx.x; i < end; i += blockDim.x) {
        float x = v[i];
        if (!isfinite(x)) {
            ++b.bad;
        } else if (x > b.v) {  // strided scan: indices rise per thread, so '>' keeps the first
            b.v = x;
            b.i = unsigned(i);
        }
    }
    b = block_best(b);
    if (threadIdx.x == 0) {
        float* o = parts + (size_t(row) * slices + slice) * 3;
        o[0] = b.v;
        o[1] = __uint_as_float(b.i);
        o[2] = __uint_as_float(b.bad);
    }
}

__global__ __launch_bounds__(256) void argmax_merge_kernel(Params a, const float* parts, int slices) {
    const int row = blockIdx.x;
    Best b{-INFINITY, 0xffffffffu, 0u};
    for (int s = threadIdx.x; s < slices; s += blockDim.x) {
        const float* o = parts + (size_t(row) * slices + s) * 3;
        b = better(b, Best{o[0], __float_as_uint(o[1]), __float_as_uint(o[2])});
    }
    b = block_best(b);
    if (threadIdx.x == 0) {
        a.p[0][2 * row] = float(b.i);
        a.p[0][2 * row + 1] = float(b.bad);
    }
}

unsigned grid_for(long n) {
    long b = (n + 255) / 256;
    return unsigned(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

}  // namespace

int run_elementwise(hipStream_t s, int op, int count, const Params& a) {
    if ((op == QR_ADD || op == QR_SILU_PRODUCT) && count % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(a.p[0]) | reinterpret_cast<uintptr_t>(a.p[1]) |
         reinterpret_cast<uintptr_t>(a.p[2])) % 16 == 0) {
        hipLaunchKernelGGL(elementwise4_kernel, dim3(grid_for(count / 4)), dim3(256), 0, s, op, count / 4, a);
        return int(hipGetLastError());
    }
    hipLaunchKernelGGL(elementwise_kernel, dim3(grid_for(count)), dim3(256), 0, s, op, count, a);
    return int(hipGetLastError());
}

// The register form when the group is 64 PER elements and every operand is
// aligned to its vector width.
template <int PER>
bool launch_rms_rows(hipStream_t s, int op, int groups, const Params& a, __bf16* planes, int width) {
    constexpr uintptr_t align = (PER >= 4 ? 4 : PER) * sizeof(float);
    const int slots[] = {0, 1, 2, 3, 4};
    const int used = op == QR_ADD_RMS_NORM ? 5 : op == QR_RMS_NORM_GATE ? 4 : 3;
    for (int k = 0; k < used; ++k)
        if (reinterpret_cast<uintptr_t>(a.p[slots[k]]) % align != 0) return false;
    if (planes && reinterpret_cast<uintptr_t>(planes) % (align / 2) != 0) return false;
    hipLaunchKernelGGL(rms_rows_kernel<PER>, dim3(ceil_div(groups, 4)), dim3(256), 0, s, op, groups, a, planes,
                       width);
    return true;
}
bool launch_rms_rows_any(hipStream_t s, int op, int groups, const Params& a, __bf16* planes, int width) {
    switch (a.n[0]) {
    case 128: return launch_rms_rows<2>(s, op, groups, a, planes, width);
    case 256: return launch_rms_rows<4>(s, op, groups, a, planes, width);
    case 512: return launch_rms_rows<8>(s, op, groups, a, planes, width);
    case 1024: return launch_rms_rows<16>(s, op, groups, a, planes, width);
    case 2048: return launch_rms_rows<32>(s, op, groups, a, planes, width);
    }
    return false;
}

int run_rms_family_planes(hipStream_t s, int op, int groups, const Params& a, __bf16* planes, int width) {
    if (op != QR_RMS_NORM && op != QR_ADD_RMS_NORM && op != QR_RMS_NORM_GATE) return int(hipErrorNotSupported);
    if (a.n[0] < 1 || width < a.n[0] || width % a.n[0] != 0 || !p3_cols_ok(width) ||
        (long(groups) * a.n[0]) % width != 0)
        return int(hipErrorNotSupported);
    if (op == QR_RMS_NORM_GATE && a.n[0] == 128) {
        const int hc = width / 128, rows = int(long(groups) / hc);
        hipLaunchKernelGGL(rms_gate_planes_kernel, dim3(unsigned((rows + 31) / 32), unsigned(hc)), dim3(256), 0, s, rows,
                           a, planes, width);
        return int(hipGetLastError());
    }
    if (!launch_rms_rows_any(s, op, groups, a, planes, width)) return int(hipErrorNotSupported);
    return int(hipGetLastError());
}

int run_rms_family(hipStream_t s, int op, int groups, const Params& a) {
    if (launch_rms_rows_any(s, op, groups, a, nullptr, a.n[0])) return int(hipGetLastError());
    if (a.n[0] <= 256)
        hipLaunchKernelGGL(rms_family_kernel<true>, dim3(ceil_div(groups, 4)), dim3(256), 0, s, op, groups, a);
    else
        hipLaunchKernelGGL(rms_family_kernel<false>, dim3(unsigned(groups)), dim3(256), 0, s, op, groups, a);
    return int(hipGetLastError());
}

int run_conv_silu(hipStream_t s, int count, const Params& a) {
    if (a.n[0] < 1 || a.n[0] > 17) return int(hipErrorInvalidValue);
    const int tokens = a.n[1] > 0 ? a.n[1] : 1;
    if (tokens <= 4) {  // decode and short verify chunks: one thread walks the tokens of its channel
        hipLaunchKernelGGL(conv_silu_kernel, dim3(ceil_div(count, 256)), dim3(256), 0, s, count, a);
        return int(hipGetLastError());
    }
    if (a.n[0] == 4)
        hipLaunchKernelGGL((conv_silu_window_kernel<4, 16>), dim3(ceil_div(count, 256), ceil_div(tokens, 16)), dim3(256),
                           0, s, count, a);
    else
        hipLaunchKernelGGL(conv_silu_tokens_kernel, dim3(ceil_div(count, 256), unsigned(tokens)), dim3(256), 0, s, count,
                           a);
    if (hipError_t e = hipGetLastError()) return int(e);
    hipLaunchKernelGGL(conv_history_kernel, dim3(ceil_div(count, 256)), dim3(256), 0, s, count, a);
    return int(hipGetLastError());
}

int run_delta_qk(hipStream_t s, int count, const Params& a) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(a.p[0]) | reinterpret_cast<uintptr_t>(a.p[1]) |
                         reinterpret_cast<uintptr_t>(a.p[2]);
    if (a.n[2] == 128 && al % 8 == 0 && a.n[3] % 2 == 0) {
        hipLaunchKernelGGL(delta_qk_pairs_kernel, dim3(ceil_div(count, 4)), dim3(256), 0, s, count, a);
        return int(hipGetLastError());
    }
    hipLaunchKernelGGL(delta_qk_kernel, dim3(ceil_div(count, 4)), dim3(256), 0, s, count, a);
    return int(hipGetLastError());
}

template <int KR, int P>
static int rule_launch(hipStream_t s, bool gated, int count, const Params& a) {
    const unsigned blocks = ceil_div(count, 4 * (64 / P));
    if (gated)
        hipLaunchKernelGGL((delta_rule_kernel<KR, P, true>), dim3(blocks), dim3(256), 0, s, count, a);
    else
        hipLaunchKernelGGL((delta_rule_kernel<KR, P, false>), dim3(blocks), dim3(256), 0, s, count, a);
    return int(hipGetLastError());
}

int run_delta_rule(hipStream_t s, bool gated, int count, const Params& a) {
    const int kd = a.n[0];
    if (kd <= 8) return rule_launch<8, 1>(s, gated, count, a);
    if (kd <= 32) return rule_launch<8, 4>(s, gated, count, a);
    if (kd <= 64) return rule_launch<16, 4>(s, gated, count, a);
    if (kd <= 128) return rule_launch<32, 4>(s, gated, count, a);
    if (kd <= 256) return rule_launch<64, 4>(s, gated, count, a);
    return int(hipErrorInvalidValue);
}

int run_attention_qkv(hipStream_t s, int op, int count, const Params& a, const float* denom) {
    if (a.n[0] > kAttnMaxHeadDim || a.n[1] > a.n[0] || a.n[1] % 2 != 0) return int(hipErrorInvalidValue);
    const dim3 waves(unsigned((count + 3) / 4));
    if (a.n[1] <= 64) {
        switch (a.n[0]) {
        case 64: hipLaunchKernelGGL(attention_qkv_wave_kernel<1>, waves, dim3(256), 0, s, op, count, a, denom); break;
        case 128: hipLaunchKernelGGL(attention_qkv_wave_kernel<2>, waves, dim3(256), 0, s, op, count, a, denom); break;
        case 256: hipLaunchKernelGGL(attention_qkv_wave_kernel<4>, waves, dim3(256), 0, s, op, count, a, denom); break;
        case 512: hipLaunchKernelGGL(attention_qkv_wave_kernel<8>, waves, dim3(256), 0, s, op, count, a, denom); break;
        default: hipLaunchKernelGGL(attention_qkv_kernel, dim3(unsigned(count)), dim3(256), 0, s, op, count, a, denom);
        }
        return int(hipGetLastError());
    }
    hipLaunchKernelGGL(attention_qkv_kernel, dim3(unsigned(count)), dim3(256), 0, s, op, count, a, denom);
    return int(hipGetLastError());
}

int run_embed(hipStream_t s, int op, int count, const Params& a) { return run_elementwise(s, op, count, a); }

// Embedding rows of a prefill chunk: the ids ride in the kernel arguments,
// kEmbedIds per launch (one block per row), so no host-to-device copy is
// queued. BF16 rows widen as EmbedBf16 does (reference.h:213-216).
constexpr int kEmbedIds = 480;
struct EmbedIds {
    int ids[kEmbedIds];
};
__global__ __launch_bounds__(256) void embed_rows_kernel(float* dst, const void* table, int width, int bf16,
                                                         EmbedIds b) {
    const size_t id = size_t(b.ids[blockIdx.x]);
    float* out = dst + size_t(blockIdx.x) * width;
    if (bf16) {
        const uint16_t* row = static_cast<const uint16_t*>(table) + id * width;
        for (int i = threadIdx.x; i < width; i += 256) out[i] = __uint_as_float(uint32_t(row[i]) << 16);
    } else {
        const float* row = static_cast<const float*>(table) + id * width;
        for (int i = threadIdx.x; i < width; i += 256) out[i] = row[i];
    }
}

int run_embed_rows(hipStream_t s, float* dst, const void* table, int width, bool bf16, const int32_t* ids, int n) {
    for (int r0 = 0; r0 < n; r0 += kEmbedIds) {
        const int m = n - r0 < kEmbedIds ? n - r0 : kEmbedIds;
        EmbedIds b{};
        for (int r = 0; r < m; ++r) b.ids[r] = ids[r0 + r];
        hipLaunchKernelGGL(embed_rows_kernel, dim3(unsigned(m)), dim3(256), 0, s, dst + size_t(r0) * width, table,
                           width, bf16 ? 1 : 0, b);
        if (hipError_t e = hipGetLastError()) return int(e);
    }
    return 0;
}

size_t argmax_parts_needed(int rows, int n) { return size_t(rows) * ceil_div(n, kArgmaxSlice) * 3; }

int run_argmax(hipStream_t s, int rows, const Params& a, float* parts, size_t parts_len) {
    const int n = a.n[0];
    const int slices = int(ceil_div(n, kArgmaxSlice));
    if (argmax_parts_needed(rows, n) > parts_len) return int(hipErrorInvalidValue);
    hipLaunchKernelGGL(argmax_slices_kernel, dim3(unsigned(slices), unsigned(rows)), dim3(256), 0, s, a, parts, slices);
    if (int e = int(hipGetLastError())) return e;
    hipLaunchKernelGGL(argmax_merge_kernel, dim3(unsigned(rows)), dim3(256), 0, s, a, parts, slices);
    return int(hipGetLastError());
}

// ---- the argmax with its slice partials in a fixed device array (no
// allocation on any call; for callers that cannot allocate). Every device the
// library runs on holds one copy of `scratch` until the process ends; every
// call on a device shares it, so calls that overlap on one device race (the
// slices kernel writes every partial the merge reads, so nothing needs
// clearing between calls). In host code `scratch` names a host-side stand-in:
// kernels get the device address that hipGetSymbolAddress returns, kept per
// device.
namespace {
static __device__ __align__(256) float scratch[kArgmaxFixedRows * (kArgmaxFixedLength / kArgmaxSlice) * 3];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int argmax_fixed_init() {
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev)) return int(e);
    if (dev < 0 || dev >= kMaxDevices) return int(hipErrorInvalidDevice);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        if (hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch))) return int(e);
        g_scratch_ptr[dev] = static_cast<float*>(ptr);
    }
    return 0;
}

int run_argmax_fixed(hipStream_t s, int rows, const Params& a) {
    const int n = a.n[0];
    if (rows < 1 || rows > kArgmaxFixedRows || n < 1 || n > kArgmaxFixedLength) return int(hipErrorInvalidValue);
    if (int e = argmax_fixed_init()) return e;
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev)) return int(e);
    float* parts = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        parts = g_scratch_ptr[dev];
    }
    constexpr size_t floats = sizeof(scratch) / sizeof(float);
    return run_argmax(s, rows, a, parts, floats);
}

}  // namespace qr
