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
    int d, heads, kv, length0, rows, span, splits;
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

// Merge the split partials: one thread per (row, head, dim).
__global__ __launch_bounds__(256) void attention_combine_kernel(ReadArgs a) {
    const long idx = blockIdx.x * long(blockDim.x) + threadIdx.x;
    const long total = long(a.rows) * a.heads * a.d;
    if (idx >= total) return;
    const int i = int(idx % a.d);
    const long rh = idx / a.d;  // row * heads + head
    const float* parts = a.parts + size_t(rh) * a.splits * (a.d + 2);
    float mm = -INFINITY;
    for (int s = 0; s < a.splits; ++s) mm = fmaxf(mm, parts[size_t(s) * (a.d + 2)]);
    float den = 0.f, num = 0.f;
    for (int s = 0; s < a.splits; ++s) {
        const float* p = parts + size_t(s) * (a.d + 2);
        const float c = p[0] == -INFINITY ? 0.f : expf(p[0] - mm);
        den += p[1] * c;
        num += p[2 + i] * c;
    }
    const size_t o = size_t(rh) * a.d + i;
    a.out[o] = (num / den) * sigmoidf_(a.gate[o]);
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

}  // namespace

size_t attention_scratch_needed(const Params& a) {
    const int tokens = a.n[5] > 0 ? a.n[5] : 1;
    if (tokens != 1) return 0;
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
    const long total = long(a.rows) * a.heads * a.d;
    hipLaunchKernelGGL(attention_combine_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, s, a);
    return int(hipGetLastError());
}

}  // namespace qr
