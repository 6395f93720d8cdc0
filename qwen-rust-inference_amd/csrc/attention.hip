// AttentionRead (op 10) on gfx950: causal GQA softmax read of the KV cache
// with the sigmoid output gate, the arithmetic of the reference's op body
// (native/rocm/reference.h:173-193): for query head h of KV head
// h / (heads / kv) and row r (length n3 + r),
//   s_p = q . k_p / sqrt(d),  out = (sum_p softmax(s)_p v_p) * sigmoid(gate).
//
// Decomposition (flash decoding): a block owns one KV head, one query row and
// one span of positions, and serves every query head of the GQA group from
// the same K/V reads. A position's d values are spread over LPP lanes (16-byte
// loads, 64/LPP positions per wave per step); scores are reduced over those
// LPP lanes; each lane keeps an online softmax (max, denominator, partial
// context) per query head. Position groups and waves are merged with the
// log-sum-exp rule. With one span the block writes the gated output; with
// several it writes (max, denominator, context) partials that a combine
// kernel merges.
#include "common.h"

namespace qr {
namespace {

struct ReadArgs {
    float* out;
    const float* query;
    const float* keys;
    const float* values;
    const float* gate;
    float* parts;  // [rows][heads][splits][d + 2] when splits > 1
    char* kpl;     // attention_prefill_bf3_kernel: K planes, [kv][tiles] blocks of B3_KBLK bytes
    char* vpl;     // ... and V^T planes, [kv][tiles] blocks of B3_VBLK bytes
    int d, heads, kv, length0, rows, span, splits, tiles;
};

template <int D, int G>
__global__ __launch_bounds__(256) void attention_read_kernel(ReadArgs a) {
    constexpr int DPL = D >= 64 ? 16 : 4;  // floats per lane
    constexpr int LPP = D / DPL;            // lanes per position
    constexpr int PPW = 64 / LPP;           // positions per wave per step
    const int split = blockIdx.x, kvh = blockIdx.y, row = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPP, slot = lane / LPP;
    const int length = a.length0 + row;
    const int begin = split * a.span, end = min(length, begin + a.span);
    const float scale = 1.f / sqrtf(float(D));
    // query vectors of the group, this lane's DPL slice
    float q[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float* qp = a.query + (size_t(row) * a.heads + size_t(kvh) * G + g) * D + sub * DPL;
#pragma unroll
        for (int e = 0; e < DPL; e += 4) {
            float4 v = *reinterpret_cast<const float4*>(qp + e);
            q[g][e] = v.x;
            q[g][e + 1] = v.y;
            q[g][e + 2] = v.z;
            q[g][e + 3] = v.w;
        }
    }
    float m[G], l[G], acc[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[g][e] = 0.f;
    }
    const size_t rowstride = size_t(a.kv) * D;
    for (int p0 = begin + wave * PPW; p0 < end; p0 += 4 * PPW) {
        const int p = p0 + slot;
        const bool live = p < end;
        float kx[DPL], vx[DPL];
        const float* kp = a.keys + size_t(live ? p : begin) * rowstride + size_t(kvh) * D + sub * DPL;
        const float* vp = a.values + size_t(live ? p : begin) * rowstride + size_t(kvh) * D + sub * DPL;
#pragma unroll
        for (int e = 0; e < DPL; e += 4) {
            float4 kv4 = *reinterpret_cast<const float4*>(kp + e);
            float4 vv4 = *reinterpret_cast<const float4*>(vp + e);
            kx[e] = kv4.x;
            kx[e + 1] = kv4.y;
            kx[e + 2] = kv4.z;
            kx[e + 3] = kv4.w;
            vx[e] = vv4.x;
            vx[e + 1] = vv4.y;
            vx[e + 2] = vv4.z;
            vx[e + 3] = vv4.w;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; ++e) s = fmaf(q[g][e], kx[e], s);
            s = group_sum<LPP>(s) * scale;
            if (live) {
                const float mn = fmaxf(m[g], s);
                const float corr = expf(m[g] - mn);  // m = -inf: 0
                const float w = expf(s - mn);
                l[g] = l[g] * corr + w;
#pragma unroll
                for (int e = 0; e < DPL; ++e) acc[g][e] = acc[g][e] * corr + w * vx[e];
                m[g] = mn;
            }
        }
    }
    // Merge the position slots of the wave (lanes with the same sub).
#pragma unroll
    for (int o = LPP; o < 64; o <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mo = __shfl_xor(m[g], o, 64), lo = __shfl_xor(l[g], o, 64);
            const float mn = fmaxf(m[g], mo);
            const float c0 = m[g] == -INFINITY ? 0.f : expf(m[g] - mn);
            const float c1 = mo == -INFINITY ? 0.f : expf(mo - mn);
            l[g] = l[g] * c0 + lo * c1;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[g][e] = acc[g][e] * c0 + __shfl_xor(acc[g][e], o, 64) * c1;
            m[g] = mn;
        }
    }
    // Merge the 4 waves through LDS: wave w's slot-0 lanes publish.
    __shared__ float sm[4][G], sl[4][G];
    __shared__ float sacc[4][G][D];
    if (slot == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (sub == 0) {
                sm[wave][g] = m[g];
                sl[wave][g] = l[g];
            }
#pragma unroll
            for (int e = 0; e < DPL; ++e) sacc[wave][g][sub * DPL + e] = acc[g][e];
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
        const int g = idx / D, i = idx % D;
        float mm = -INFINITY;
        for (int w = 0; w < 4; ++w) mm = fmaxf(mm, sm[w][g]);
        float den = 0.f, num = 0.f;
        for (int w = 0; w < 4; ++w) {
            const float c = sm[w][g] == -INFINITY ? 0.f : expf(sm[w][g] - mm);
            den += sl[w][g] * c;
            num += sacc[w][g][i] * c;
        }
        const int head = kvh * G + g;
        if (a.splits == 1) {
            const size_t o = (size_t(row) * a.heads + head) * D + i;
            a.out[o] = (num / den) * sigmoidf_(a.gate[o]);
        } else {
            float* part = a.parts + ((size_t(row) * a.heads + head) * a.splits + split) * (D + 2);
            if (i == 0) {
                part[0] = mm;
                part[1] = den;
            }
            part[2 + i] = num;
        }
    }
}

// Merge the split partials: LANES lanes (1, or the 4 of a quad) per (row,
// head, 4 dims), lane q taking splits q, q + LANES, ... and a quad's (max,
// sum, weighted sums) combined by two xor shuffles. Quads for a decode row
// (tens of splits: each lane's loads in flight together), one lane for a
// prefill chunk (a few shares: more lanes only add shuffles). The partial
// sums are read as 8-byte pairs (a partial is d + 2 floats: even, not a
// multiple of 4). The order of every sum is fixed for a given split count.
template <int LANES>
__global__ __launch_bounds__(256) void attention_combine_kernel(ReadArgs a) {
    typedef float f2v __attribute__((ext_vector_type(2)));
    typedef float f4v __attribute__((ext_vector_type(4)));
    static_assert(LANES == 1 || LANES == 4 || LANES == 16, "one lane, a quad or 16 lanes");
    const long idx = blockIdx.x * long(blockDim.x) + threadIdx.x;
    const int q = a.d / 4;
    const long total = long(a.rows) * a.heads * q * LANES;  // whole quads: the shuffles see only live lanes
    if (idx >= total) return;
    const int lq = int(idx % LANES);
    const long e = idx / LANES;
    const int i = 4 * int(e % q);
    const long rh = e / q;  // row * heads + head
    const float* parts = a.parts + size_t(rh) * a.splits * (a.d + 2);
    float mm = -INFINITY;
#pragma unroll 8
    for (int s = lq; s < a.splits; s += LANES) mm = fmaxf(mm, parts[size_t(s) * (a.d + 2)]);
#pragma unroll
    for (int o = 1; o < LANES; o <<= 1) mm = fmaxf(mm, __shfl_xor(mm, o, 64));
    float den = 0.f;
    f4v num = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int s = lq; s < a.splits; s += LANES) {
        const float* p = parts + size_t(s) * (a.d + 2);
        const float c = p[0] == -INFINITY ? 0.f : expf(p[0] - mm);
        den += p[1] * c;
        const f2v lo = *reinterpret_cast<const f2v*>(p + 2 + i), hi = *reinterpret_cast<const f2v*>(p + 4 + i);
        num.x += lo.x * c;
        num.y += lo.y * c;
        num.z += hi.x * c;
        num.w += hi.y * c;
    }
    if constexpr (LANES > 1) {
#pragma unroll
        for (int o = 1; o < LANES; o <<= 1) {
            den += __shfl_xor(den, o, 64);
            num.x += __shfl_xor(num.x, o, 64);
            num.y += __shfl_xor(num.y, o, 64);
            num.z += __shfl_xor(num.z, o, 64);
            num.w += __shfl_xor(num.w, o, 64);
        }
        if (lq != 0) return;
    }
    const size_t o = size_t(rh) * a.d + i;
    const f4v g = *reinterpret_cast<const f4v*>(a.gate + o);
    f4v r;
    r.x = (num.x / den) * sigmoidf_(g.x);
    r.y = (num.y / den) * sigmoidf_(g.y);
    r.z = (num.z / den) * sigmoidf_(g.z);
    r.w = (num.w / den) * sigmoidf_(g.w);
    *reinterpret_cast<f4v*>(a.out + o) = r;
}
// Launch of the merge: quads from 16 splits on, 16 lanes per group from 64
// (a decode row has only rows x heads x d / 4 groups: 512 at the 0.8B shape,
// so with one lane or a quad each lane walks many splits in turn).
int launch_combine(hipStream_t s, const ReadArgs& a) {
    const long groups = long(a.rows) * a.heads * (a.d / 4);
    if (a.splits >= 64)
        hipLaunchKernelGGL(attention_combine_kernel<16>, dim3(ceil_div(groups * 16, 256)), dim3(256), 0, s, a);
    else if (a.splits >= 16)
        hipLaunchKernelGGL(attention_combine_kernel<4>, dim3(ceil_div(groups * 4, 256)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(attention_combine_kernel<1>, dim3(ceil_div(groups, 256)), dim3(256), 0, s, a);
    return int(hipGetLastError());
}

// ---------------------------------------------------------------- prefill
// Prefill rows (flash attention on fp32 MFMA, v_mfma_f32_32x32x2_f32): a block
// owns 32 consecutive query rows and one KV head; wave w serves query head
// kv * G + w, so each K / V tile staged in LDS feeds the whole GQA group.
// Per tile of 32 positions a wave forms S^T = K Q^T (32 positions x 32
// queries: lane l holds 16 scores of query l % 32), keeps the online softmax
// per query in registers (the two lane halves of a query combine with one
// shuffle), and accumulates O^T += V^T P^T, whose B operand is the score
// accumulator itself (step st of the product uses the position that score
// register st holds). Q^T stays in registers (D / 2 per lane), O^T in
// accumulators (D / 2 per lane). The next tile's K / V are loaded into
// registers while the current one is multiplied. Positions past the block's
// last visible one are zero-filled; scores past a row's own length are -inf.
// KV split (blockIdx.z of a.splits): when there are too few (query tile, KV
// head) blocks to fill the CUs, each block takes an equal share of its tile's
// K / V tiles and writes (max, sum, unnormalised context) partials that
// attention_combine_kernel merges, as for a decode row.
template <int D>
struct PrefillShape {
    static constexpr int DH = D / 2;                    // score steps (dims hl * DH + st)
    static constexpr int SKEW = DH % 64 == 0 ? 32 : 0;  // upper dim half 32 banks over
    static constexpr int KS = D + 33;                   // K row stride (= 33 mod 64)
    static constexpr int VS = D + 8;                    // V row stride (4 rows = 32 banks)
    static constexpr int DT = D / 32;                   // output dim tiles
};

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int acc_row(int r, int hl) { return 8 * (r >> 2) + 4 * hl + (r & 3); }

// Scheduling of a run of N MFMAs, each with one LDS operand read: four reads
// ahead, then one read per MFMA, so the reads are neither serialised behind
// their MFMAs nor all hoisted (which would hold N operands in registers).
template <int N>
__device__ __forceinline__ void pipeline_ds_mfma() {
#pragma unroll
    for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int i = 0; i < N - 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
}

// (D, G) with the prefill kernel: at most 8 float4 of K (and of V) per thread
// per tile, and, at 512 threads (a 256-register budget), D <= 128.
constexpr bool prefill_shape_ok(int d, int g) { return d / (8 * g) <= 8 && (g < 8 || d <= 128); }

template <int D, int G>
__global__ __launch_bounds__(64 * G) void attention_prefill_kernel(ReadArgs a) {
    using S = PrefillShape<D>;
    constexpr int T = 64 * G, F4 = 32 * D / 4 / T;  // float4 of K (and of V) per thread per tile
    static_assert(F4 >= 1 && (32 * D / 4) % T == 0, "tile load split");
    __shared__ float ks[2][32 * S::KS], vs[2][32 * S::VS];
    const int qtiles = (a.rows + 31) / 32;
    const int q0 = (qtiles - 1 - int(blockIdx.x)) * 32, kvh = blockIdx.y;  // longest rows first
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, lc = lane & 31, hl = lane >> 5;
    const int head = kvh * G + w, qrow = q0 + lc;
    const int len = a.length0 + qrow;  // positions [0, len) visible to this lane's query
    const int len_max = a.length0 + min(a.rows, q0 + 32) - 1;
    const int all_tiles = (len_max + 31) / 32, share = (all_tiles + a.splits - 1) / a.splits;
    const int t_begin = int(blockIdx.z) * share, t_end = min(all_tiles, t_begin + share);
    if (t_begin >= t_end) {  // an empty share (early query tiles): a neutral partial
        if (qrow < a.rows) {
            float* part = a.parts + ((size_t(qrow) * a.heads + head) * a.splits + blockIdx.z) * (D + 2);
            for (int i = hl; i < D + 2; i += 2) part[i] = i == 0 ? -INFINITY : 0.f;
        }
        return;
    }
    const float scale = 1.f / sqrtf(float(D));
    const size_t rowstride = size_t(a.kv) * D;
    float qv[S::DH];
    {
        const float* qp = a.query + (size_t(qrow) * a.heads + head) * D + hl * S::DH;
#pragma unroll
        for (int e = 0; e < S::DH; e += 4) {
            const f4v v = qrow < a.rows ? *reinterpret_cast<const f4v*>(qp + e) : f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) qv[e + j] = v[j];
        }
    }
    f4v kp[F4], vp[F4];
    auto fetch = [&](int t) {
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int e = int(threadIdx.x) + T * i, pos = t * 32 + e / (D / 4), c = (e % (D / 4)) * 4;
            const size_t off = size_t(pos) * rowstride + size_t(kvh) * D + c;
            const bool live = pos < len_max;
            kp[i] = live ? *reinterpret_cast<const f4v*>(a.keys + off) : f4v{0.f, 0.f, 0.f, 0.f};
            vp[i] = live ? *reinterpret_cast<const f4v*>(a.values + off) : f4v{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int e = int(threadIdx.x) + T * i, pr = e / (D / 4), c = (e % (D / 4)) * 4;
            float* kd = &ks[buf][pr * S::KS + c + (c >= S::DH ? S::SKEW : 0)];
            float* vd = &vs[buf][pr * S::VS + c];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kd[j] = kp[i][j];
                vd[j] = vp[i][j];
            }
        }
    };
    fetch(t_begin);
    stage(t_begin & 1);
    __syncthreads();
    f16v o[S::DT];
#pragma unroll
    for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
    float m = -INFINITY, l = 0.f;
    for (int t = t_begin; t < t_end; ++t) {
        const int buf = t & 1;
        if (t + 1 < t_end) fetch(t + 1);
        const float* kt = &ks[buf][lc * S::KS + hl * (S::DH + S::SKEW)];
        f16v sc;
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = 0.f;
#pragma unroll
        for (int st = 0; st < S::DH; ++st) sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kt[st], qv[st], sc, 0, 0, 0);
        pipeline_ds_mfma<S::DH>();
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float v = t * 32 + acc_row(r, hl) < len ? sc[r] * scale : -INFINITY;
            sc[r] = v;
            mx = fmaxf(mx, v);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // -inf while a row has seen no visible position (a KV share past its length)
        const float mn = fmaxf(m, mx), mref = mn == -INFINITY ? 0.f : mn;
        const float corr = expf(m - mref);
        m = mn;
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = expf(sc[r] - mref);
            sc[r] = p;
            ps += p;
        }
        l = l * corr + ps;
        const float* vt = &vs[buf][lc];
#pragma unroll
        for (int dt = 0; dt < S::DT; ++dt) {
            o[dt] *= corr;
#pragma unroll
            for (int st = 0; st < 16; ++st)
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt[acc_row(st, hl) * S::VS + dt * 32], sc[st], o[dt], 0,
                                                             0, 0);
        }
        pipeline_ds_mfma<16 * S::DT>();
        if (t + 1 < t_end) stage(buf ^ 1);
        __syncthreads();
    }
    const float den = l + __shfl_xor(l, 32, 64);
    if (qrow < a.rows && a.splits == 1) {
        const size_t base = (size_t(qrow) * a.heads + head) * D;
#pragma unroll
        for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const size_t idx = base + dt * 32 + acc_row(r, hl);
                a.out[idx] = (o[dt][r] / den) * sigmoidf_(a.gate[idx]);
            }
    } else if (qrow < a.rows) {
        float* part = a.parts + ((size_t(qrow) * a.heads + head) * a.splits + blockIdx.z) * (D + 2);
        if (hl == 0) {
            part[0] = m;
            part[1] = den;
        }
#pragma unroll
        for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) part[2 + dt * 32 + acc_row(r, hl)] = o[dt][r];
    }
}

// ---- D = 256, G = 4 (the attention layers of the Qwen3.5-0.8B shape): the
// block / share decomposition, masking and online softmax of
// attention_prefill_kernel, with both products on BF16 MFMA
// (v_mfma_f32_32x32x16_bf16) over operands split into three BF16 parts each
// (x = x0 + x1 + x2, the six part products with p + q <= 2 summed smallest
// first: fp32 accuracy, as the prefill GEMM) at 2.7x the rate of the fp32
// MFMA.
// 8 waves: wave w is query head w % 4 of the group over dims 128 (w / 4) ..
// + 127 (its half). S^T = K Q^T over the half: A = the tile's K rows (three
// planes in LDS), B = Q^T (three planes in registers, split once); the two
// halves' partial scores are exchanged through LDS and added (the same sum
// on both waves), so both run the same softmax. O^T += V^T P^T over the
// half's dims: A = V^T (three planes in LDS, transposed), B = P^T taken
// straight from the score accumulator: lane l holds keys 8 (r / 4) +
// 4 (l / 32) + r % 4 of its query in register r, so MFMA k index 8 (l / 32)
// + e of step s is key 16 s + 8 (e / 4) + 4 (l / 32) + e % 4 when the B
// operand of step s is registers 8 s .. 8 s + 7; V^T keeps its key positions
// in that order (bits 2 and 3 of the key swapped), so no value crosses
// lanes.
// The three BF16 planes of K and of V^T are made once per call, before the
// attention kernel, by kv_planes_kernel (every block re-splitting its KV
// head's rows would repeat the split n / 32 times), in exactly the LDS layout
// of one tile: K 3 x 32 x 264 (rows padded so the 16-byte operand reads of 8
// consecutive lanes hit distinct banks) and V^T 3 x 256 x 40 with its key
// positions in the score accumulator's order (below), each tile block padded
// to whole 8 KiB rounds of 16-byte LDS DMA (56 and 64 KiB). The attention
// kernel stages a tile by LDS DMA (global_load_lds_dwordx4: 64 lanes x 16 B
// straight into LDS, no registers): each of the 8 waves issues 7 K and 8 V
// instructions. The loop runs one tile ahead on the score product: tile t + 1's
// scores are multiplied while tile t's softmax runs, then tile t's PV product;
// K of tile t + 2 is loaded during that PV product (every wave is past its
// reads of tile t + 1's K), and V of tile t + 1 during the next score product
// (every wave is past its reads of tile t's V), so one K buffer and one V
// buffer suffice (56 + 64 + 32 KiB score exchange = 152 KiB) and the barriers
// wait for LDS only, never for loads in flight.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
constexpr int B3_KROW = 256 + 8, B3_VROW = 40;
constexpr int B3_KBLK = 56 * 1024, B3_VBLK = 64 * 1024;  // bytes per tile (3 x 32 x 264 and 3 x 256 x 40 BF16, padded)
constexpr int B3_KDMA = B3_KBLK / 8192, B3_VDMA = B3_VBLK / 8192;  // DMA instructions per wave per tile

struct Split3 {
    __bf16 h[3];
};
__device__ __forceinline__ Split3 split3(float x) {
    Split3 o;
    o.h[0] = __bf16(x);
    const float r1 = x - float(o.h[0]);
    o.h[1] = __bf16(r1);
    o.h[2] = __bf16(r1 - float(o.h[1]));
    return o;
}
// the V^T position of tile key k: bits 2 and 3 swapped
__device__ __forceinline__ int vpos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

// One block per (tile of 32 positions, KV head): K and V rows of positions
// [32 t, 32 t + 32) split into their planes; positions at or past `len` (no
// query sees them) and the padding are zero.
__global__ __launch_bounds__(256) void kv_planes_kernel(ReadArgs a, int len) {
    constexpr int D = 256;
    const int t = int(blockIdx.x), kvh = int(blockIdx.y), tid = int(threadIdx.x);
    const size_t rowstride = size_t(a.kv) * D, blk = size_t(kvh) * a.tiles + t;
    __bf16* kb = reinterpret_cast<__bf16*>(a.kpl + blk * B3_KBLK);
    __bf16* vb = reinterpret_cast<__bf16*>(a.vpl + blk * B3_VBLK);
    const f4v z = {0.f, 0.f, 0.f, 0.f};
    f4v kv[8], vv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // K: key f / 64, dims 4 (f % 64)
        const int f = tid + 256 * i, pos = 32 * t + (f >> 6), c = (f & 63) * 4;
        kv[i] = pos < len ? *reinterpret_cast<const f4v*>(a.keys + size_t(pos) * rowstride + size_t(kvh) * D + c) : z;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // V: key quad b % 8, dim quad b / 8
        const int b = tid + 256 * i, kq = b & 7, cq = b >> 3;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int pos = 32 * t + 4 * kq + r;
            vv[4 * i + r] = pos < len ? *reinterpret_cast<const f4v*>(a.values + size_t(pos) * rowstride +
                                                                      size_t(kvh) * D + 4 * cq)
                                      : z;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int f = tid + 256 * i, key = f >> 6, c = (f & 63) * 4;
        bf16x4 h[3];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const Split3 x = split3(kv[i][e]);
#pragma unroll
            for (int p = 0; p < 3; ++p) h[p][e] = x.h[p];
        }
#pragma unroll
        for (int p = 0; p < 3; ++p) *reinterpret_cast<bf16x4*>(kb + (p * 32 + key) * B3_KROW + c) = h[p];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int b = tid + 256 * i, kq = b & 7, cq = b >> 3, p0 = vpos(4 * kq);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            bf16x4 h[3];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const Split3 x = split3(vv[4 * i + r][d]);
#pragma unroll
                for (int p = 0; p < 3; ++p) h[p][r] = x.h[p];
            }
#pragma unroll
            for (int p = 0; p < 3; ++p) *reinterpret_cast<bf16x4*>(vb + (p * D + 4 * cq + d) * B3_VROW + p0) = h[p];
        }
    }
    // padding: K row ends (96 x 16 B) and tail, V^T row ends (768 x 16 B) and tail
    const bf16x8 zb = {};
    if (tid < 96) *reinterpret_cast<bf16x8*>(kb + tid * B3_KROW + 256) = zb;
    for (int e = 3 * 32 * B3_KROW + 8 * tid; e < B3_KBLK / 2; e += 8 * 256) *reinterpret_cast<bf16x8*>(kb + e) = zb;
    for (int r = tid; r < 3 * D; r += 256) *reinterpret_cast<bf16x8*>(vb + r * B3_VROW + 32) = zb;
    for (int e = 3 * D * B3_VROW + 8 * tid; e < B3_VBLK / 2; e += 8 * 256) *reinterpret_cast<bf16x8*>(vb + e) = zb;
}

// LDS barrier that leaves the DMA loads in flight: LDS operations done
// (lgkmcnt(0)), then s_barrier.
__device__ __forceinline__ void b3_lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Waits until at most N vector memory operations of this wave are in flight
// (lgkmcnt and expcnt not waited).
template <int N>
__device__ __forceinline__ void b3_vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// This wave's N DMA instructions of one tile block: 1 KiB each, instruction i
// of wave w copies bytes 1 KiB (8 i + w) .. + 1023 (M0 = the LDS byte address,
// lane l's 16 bytes land at M0 + 16 l). Written as inline assembly so that
// the compiler, which cannot tell which LDS array an LDS DMA writes, does not
// wait for every one in flight before each LDS read: the kernel orders them
// itself (b3_vm_wait before the barrier that publishes a tile).
template <int N>
__device__ __forceinline__ void b3_dma(const char* src, const void* dst, int w, int lane) {
    const unsigned lds = unsigned(reinterpret_cast<size_t>((__attribute__((address_space(3))) const char*)dst));
    const unsigned voff = unsigned(lane) * 16u;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int c = 8 * i + w;
        const char* base = src + c * 1024;
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, %2" ::"v"(voff), "s"(lds + unsigned(c) * 1024u),
                     "s"(base)
                     : "memory", "m0");
    }
}

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_prefill_bf3_kernel(
    ReadArgs a) {
    constexpr int D = 256, G = 4, HALF = D / 2, DT = HALF / 32;
    __shared__ __attribute__((aligned(16))) __bf16 ks[B3_KBLK / 2];  // [3][32][B3_KROW] + DMA padding
    __shared__ __attribute__((aligned(16))) __bf16 vt[B3_VBLK / 2];  // [3][D][B3_VROW] + DMA padding
    __shared__ float xch[8][16][64];
    const int qtiles = (a.rows + 31) / 32;
    const int q0 = (qtiles - 1 - int(blockIdx.x)) * 32, kvh = blockIdx.y;  // longest rows first
    const int tid = int(threadIdx.x), lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), lc = lane & 31,
              hl = lane >> 5;
    const int g = w & 3, dh = w >> 2, d0 = dh * HALF;
    const int head = kvh * G + g, qrow = q0 + lc;
    const int len = a.length0 + qrow;  // positions [0, len) visible to this lane's query
    const int len_max = a.length0 + min(a.rows, q0 + 32) - 1;
    const int all_tiles = (len_max + 31) / 32, share = (all_tiles + a.splits - 1) / a.splits;
    const int t_begin = int(blockIdx.z) * share, t_end = min(all_tiles, t_begin + share);
    if (t_begin >= t_end) {  // an empty share (early query tiles): a neutral partial
        if (qrow < a.rows && dh == 0) {
            float* part = a.parts + ((size_t(qrow) * a.heads + head) * a.splits + blockIdx.z) * (D + 2);
            for (int i = hl; i < D + 2; i += 2) part[i] = i == 0 ? -INFINITY : 0.f;
        }
        return;
    }
    const float scale = 1.f / sqrtf(float(D));
    const char* kblk = a.kpl + size_t(kvh) * a.tiles * B3_KBLK;
    const char* vblk = a.vpl + size_t(kvh) * a.tiles * B3_VBLK;
    bf16x8 qb[3][8];  // Q^T planes: step s, element e = dim d0 + 16 s + 8 hl + e of this lane's query
    {
        const float* qp = a.query + (size_t(qrow) * a.heads + head) * D + d0 + 8 * hl;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const f4v z = {0.f, 0.f, 0.f, 0.f};
            const f4v v0 = qrow < a.rows ? *reinterpret_cast<const f4v*>(qp + 16 * s) : z;
            const f4v v1 = qrow < a.rows ? *reinterpret_cast<const f4v*>(qp + 16 * s + 4) : z;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const Split3 x = split3(e < 4 ? v0[e] : v1[e - 4]);
#pragma unroll
                for (int p = 0; p < 3; ++p) qb[p][s][e] = x.h[p];
            }
        }
    }
    constexpr int P[6] = {2, 1, 0, 1, 0, 0}, Q[6] = {0, 1, 2, 0, 1, 0};  // part products, smallest first
    // this wave's partial scores of the tile in ks (its half of the dims)
    auto scores = [&](f16v& sc) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            bf16x8 ka[3];
#pragma unroll
            for (int p = 0; p < 3; ++p)
                ka[p] = *reinterpret_cast<const bf16x8*>(&ks[(p * 32 + lc) * B3_KROW + d0 + 16 * s + 8 * hl]);
#pragma unroll
            for (int pq = 0; pq < 6; ++pq) sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[P[pq]], qb[Q[pq]][s], sc, 0, 0, 0);
        }
    };
    // partial + the partner's (exchanged in xch) = the tile's scaled scores,
    // -inf at positions this lane's query does not see
    auto finish = [&](f16v& sc, int t) {
        if (t * 32 + 31 < a.length0 + q0) {  // every key of the tile visible to every query of the block
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[r] = (sc[r] + xch[w ^ 4][r][lane]) * scale;  // (addition commutes: same on both)
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float full = sc[r] + xch[w ^ 4][r][lane];
                sc[r] = t * 32 + acc_row(r, hl) < len ? full * scale : -INFINITY;
            }
        }
    };
    b3_dma<B3_KDMA>(kblk + size_t(t_begin) * B3_KBLK, ks, w, lane);
    b3_dma<B3_VDMA>(vblk + size_t(t_begin) * B3_VBLK, vt, w, lane);
    b3_vm_wait<B3_VDMA>();  // this wave's K instructions done
    b3_lds_barrier();
    f16v sc, scn;
    scores(sc);
#pragma unroll
    for (int r = 0; r < 16; ++r) xch[w][r][lane] = sc[r];
    b3_lds_barrier();  // scores exchanged; every wave is past its K reads
    if (t_begin + 1 < t_end) b3_dma<B3_KDMA>(kblk + size_t(t_begin + 1) * B3_KBLK, ks, w, lane);
    finish(sc, t_begin);
    if (t_begin + 1 < t_end) {
        b3_vm_wait<0>();   // tile t_begin + 1's K (and t_begin's V) landed
        b3_lds_barrier();  // ... for every wave; every wave past its xch reads
    }
    f16v o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
    float m = -INFINITY, l = 0.f;
    // Software-pipelined by one tile: at the top of iteration t, sc holds tile
    // t's scores, tile t + 1's K is in ks (if any), tile t's V is in flight to
    // vt. Tile t + 1's score product (MFMA) and tile t's softmax (VALU) are
    // independent and share one basic block, so they issue interleaved.
    for (int t = t_begin; t < t_end; ++t) {
        const bool more = t + 1 < t_end;
        // tile t + 1's partial scores (the last tile multiplies stale K: unused)
        scores(scn);
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // -inf while a row has seen no visible position (a KV share past its length)
        const float mn = fmaxf(m, mx), mref = mn == -INFINITY ? 0.f : mn;
        // the hardware exponential (v_exp_f32 of x log2 e): arguments are <= 0,
        // where its error (a few ulp, plus |x| 2^-24 from the scaling) stays far
        // below the fp32 bound the outputs are held to; exp(-inf) = 0
        const float corr = __expf(m - mref);
        m = mn;
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sc[r] = __expf(sc[r] - mref);
            ps += sc[r];
        }
        l = l * corr + ps;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] *= corr;  // exact when the maximum did not move (corr = 1)
        // the softmax is computed here, beside the score product's MFMAs (the
        // compiler would otherwise sink it to the PV product after the barrier)
        asm volatile("" : "+v"(sc), "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]), "+v"(l));
        if (more)
#pragma unroll
            for (int r = 0; r < 16; ++r) xch[w][r][lane] = scn[r];
        b3_vm_wait<0>();   // tile t's V landed (the only load in flight)
        b3_lds_barrier();  // ... for every wave; tile t + 1's partials exchanged; every wave past its K reads
        if (t + 2 < t_end) b3_dma<B3_KDMA>(kblk + size_t(t + 2) * B3_KBLK, ks, w, lane);
        if (more) finish(scn, t + 1);
        // key steps outermost, so one step's P^T planes are live at a time
        // (each accumulator still takes step 0's products, then step 1's)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            bf16x8 pb[3];  // P^T planes of step s: element e = register 8 s + e
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const Split3 x = split3(sc[8 * s + e]);
#pragma unroll
                for (int p = 0; p < 3; ++p) pb[p][e] = x.h[p];
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                bf16x8 va[3];
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    va[p] = *reinterpret_cast<const bf16x8*>(
                        &vt[(p * D + d0 + 32 * dt + lc) * B3_VROW + 16 * s + 8 * hl]);
#pragma unroll
                for (int pq = 0; pq < 6; ++pq)
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[P[pq]], pb[Q[pq]], o[dt], 0, 0, 0);
            }
        }
        if (more) {
            b3_vm_wait<0>();   // tile t + 2's K landed (if it was issued)
            b3_lds_barrier();  // ... for every wave, and every wave is past its V reads and xch reads
            b3_dma<B3_VDMA>(vblk + size_t(t + 1) * B3_VBLK, vt, w, lane);
            sc = scn;
        }
    }
    const float den = l + __shfl_xor(l, 32, 64);
    if (qrow < a.rows && a.splits == 1) {
        const size_t base = (size_t(qrow) * a.heads + head) * D + d0;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const size_t idx = base + dt * 32 + acc_row(r, hl);
                a.out[idx] = (o[dt][r] / den) * sigmoidf_(a.gate[idx]);
            }
    } else if (qrow < a.rows) {
        float* part = a.parts + ((size_t(qrow) * a.heads + head) * a.splits + blockIdx.z) * (D + 2);
        if (hl == 0 && dh == 0) {
            part[0] = m;
            part[1] = den;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) part[2 + d0 + dt * 32 + acc_row(r, hl)] = o[dt][r];
    }
}

template <int D, int G>
int launch_prefill_g(hipStream_t s, const ReadArgs& a) {
    if constexpr (prefill_shape_ok(D, G)) {
        const dim3 grid(ceil_div(a.rows, 32), unsigned(a.kv), unsigned(a.splits));
        if constexpr (D == 256 && G == 4) {
            hipLaunchKernelGGL(kv_planes_kernel, dim3(unsigned(a.tiles), unsigned(a.kv)), dim3(256), 0, s, a,
                               a.length0 + a.rows - 1);
            hipLaunchKernelGGL(attention_prefill_bf3_kernel, grid, dim3(512), 0, s, a);
        } else
            hipLaunchKernelGGL((attention_prefill_kernel<D, G>), grid, dim3(64 * G), 0, s, a);
        if (a.splits == 1) return int(hipGetLastError());
        if (hipError_t e = hipGetLastError()) return int(e);
        return launch_combine(s, a);
    }
    return int(hipErrorInvalidValue);
}
template <int D>
int launch_prefill(hipStream_t s, const ReadArgs& a, int group) {
    switch (group) {
    case 1: return launch_prefill_g<D, 1>(s, a);
    case 2: return launch_prefill_g<D, 2>(s, a);
    case 4: return launch_prefill_g<D, 4>(s, a);
    case 8: return launch_prefill_g<D, 8>(s, a);
    }
    return int(hipErrorInvalidValue);
}

template <int D>
int launch_d(hipStream_t s, const ReadArgs& a, int group) {
    dim3 grid(unsigned(a.splits), unsigned(a.kv), unsigned(a.rows));
    switch (group) {
    case 1: hipLaunchKernelGGL((attention_read_kernel<D, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attention_read_kernel<D, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attention_read_kernel<D, 4>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((attention_read_kernel<D, 8>), grid, dim3(256), 0, s, a); break;
    default: return int(hipErrorInvalidValue);
    }
    return int(hipGetLastError());
}

// Splits for one decode row: about 512 blocks over the KV heads, spans a
// multiple of 16 positions.
int decode_splits(int length, int kv, int& span) {
    const int target = 512 / (kv > 0 ? kv : 1);
    int s = (length + target - 1) / target;
    s = (s + 15) / 16 * 16;
    if (s < 16) s = 16;
    span = s;
    return (length + s - 1) / s;
}

constexpr int kPrefillMinRows = 8;  // fewer rows (decode, verify): attention_read_kernel

bool prefill_path(int d, int group, int rows) {
    return rows >= kPrefillMinRows && (d == 64 || d == 128 || d == 256) &&
           (group == 1 || group == 2 || group == 4 || group == 8) && prefill_shape_ok(d, group);
}
// KV splits of a prefill chunk: about 512 blocks, at most 8 shares per tile.
int prefill_splits(int rows, int kv) {
    const long blocks = long(ceil_div(rows, 32)) * (kv > 0 ? kv : 1);
    long s = (512 + blocks - 1) / blocks;
    return int(s < 1 ? 1 : s > 8 ? 8 : s);
}

// Scratch of a prefill call, in floats: the split partials, then (head dim
// 256, 4 query heads per KV head) the K and V^T planes at a 256-byte boundary.
size_t prefill_parts_floats(int tokens, int heads, int kv, int d) {
    const int splits = prefill_splits(tokens, kv);
    return splits > 1 ? (size_t(tokens) * heads * splits * (d + 2) + 63) / 64 * 64 : 0;
}
int prefill_tiles(int length0, int tokens) { return ceil_div(length0 + tokens - 1, 32); }

}  // namespace

size_t attention_scratch_needed(const Params& a) {
    const int tokens = a.n[5] > 0 ? a.n[5] : 1;
    const int group = a.n[2] > 0 ? a.n[1] / a.n[2] : 0;
    if (tokens > 1) {
        if (!prefill_path(a.n[0], group, tokens)) return 0;
        size_t need = prefill_parts_floats(tokens, a.n[1], a.n[2], a.n[0]);
        if (a.n[0] == 256 && group == 4)
            need += size_t(a.n[2]) * prefill_tiles(a.n[3], tokens) * (B3_KBLK + B3_VBLK) / sizeof(float);
        return need;
    }
    int span;
    const int splits = decode_splits(a.n[3], a.n[2], span);
    return splits > 1 ? size_t(a.n[1]) * splits * (a.n[0] + 2) : 0;
}

int run_attention_read(hipStream_t s, int heads_count, const Params& p, float* scratch, size_t scratch_len) {
    ReadArgs a{};
    a.out = p.p[0];
    a.query = p.p[1];
    a.keys = p.p[2];
    a.values = p.p[3];
    a.gate = p.p[4];
    a.d = p.n[0];
    a.heads = p.n[1];
    a.kv = p.n[2];
    a.length0 = p.n[3];
    a.rows = p.n[5] > 0 ? p.n[5] : 1;
    const int group = a.kv > 0 ? a.heads / a.kv : 0;
    if (a.kv < 1 || a.heads % a.kv != 0 || heads_count != a.heads || a.length0 < 1) return int(hipErrorInvalidValue);
    if (a.rows == 1) {
        a.splits = decode_splits(a.length0, a.kv, a.span);
        if (a.splits > 1) {
            if (size_t(a.heads) * a.splits * (a.d + 2) > scratch_len) return int(hipErrorInvalidValue);
            a.parts = scratch;
        }
    } else {
        a.splits = 1;
        a.span = a.length0 + a.rows;  // row r reads its own length inside the span
    }
    if (prefill_path(a.d, group, a.rows)) {
        a.splits = prefill_splits(a.rows, a.kv);
        const size_t parts = prefill_parts_floats(a.rows, a.heads, a.kv, a.d);
        if (parts > scratch_len) return int(hipErrorInvalidValue);
        if (a.splits > 1) a.parts = scratch;
        if (a.d == 256 && group == 4) {
            a.tiles = prefill_tiles(a.length0, a.rows);
            const size_t planes = size_t(a.kv) * a.tiles * (B3_KBLK + B3_VBLK) / sizeof(float);
            if (parts + planes > scratch_len) return int(hipErrorInvalidValue);
            a.kpl = reinterpret_cast<char*>(scratch + parts);
            a.vpl = a.kpl + size_t(a.kv) * a.tiles * B3_KBLK;
        }
        switch (a.d) {
        case 64: return launch_prefill<64>(s, a, group);
        case 128: return launch_prefill<128>(s, a, group);
        default: return launch_prefill<256>(s, a, group);
        }
    }
    int e;
    switch (a.d) {
    case 4: e = launch_d<4>(s, a, group); break;
    case 8: e = launch_d<8>(s, a, group); break;
    case 16: e = launch_d<16>(s, a, group); break;
    case 32: e = launch_d<32>(s, a, group); break;
    case 64: e = launch_d<64>(s, a, group); break;
    case 128: e = launch_d<128>(s, a, group); break;
    case 256: e = launch_d<256>(s, a, group); break;
    default: return int(hipErrorInvalidValue);
    }
    if (e || a.splits == 1) return e;
    return launch_combine(s, a);
}

}  // namespace qr
