// qr_delta_mixer for one token (decode) on gfx950: ConvSilu, DeltaQk,
// DeltaRuleGated and RmsNormGate (offset 0) of one Gated DeltaNet layer in a
// single launch, with the outputs the four ops write (reference
// native/rocm/bridge.cpp:730-796 for the contract; the arithmetic of each
// step is reference.h:96-116, 134-143, 48-60 + 149-170, 201-207).
//
// One block per value head, 512 threads:
//   1. conv + SiLU of the head's q, k and v channels (one channel per thread,
//      history oldest -> newest updated in place);
//   2. L2 norms of q and k (block reductions); q / sqrt(dk);
//   3. gates g = -exp(A_log) softplus(a + dt), beta = sigmoid(b);
//   4. the rule on the head's [dk, dv] state: 4 lanes per value column, 32
//      key rows each in VGPRs, column sums over the 4 lanes by two shuffles;
//   5. gated RMSNorm of the head's dv outputs with silu(z).
// Shape: key_heads == value_heads, dk == 128, dv == 128, kernel <= 8.
#include "common.h"

namespace qr {
namespace {

constexpr int kDk = 128, kDv = 128, kThreads = 512, kP = 4, kKR = kDk / kP;

__global__ __launch_bounds__(kThreads) void delta_mixer_decode_kernel(QrDelta d) {
    __shared__ float qs[kDk], ks[kDk], vs[kDv], core[kDv];
    __shared__ float red[16];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int K = d.kernel, kd = d.key_heads * kDk;
    // 1. conv + SiLU: channels q [h*dk, +dk), k [kd + h*dk, +dk), v [2kd + h*dv, +dv)
    if (tid < kDk + kDk + kDv) {
        int ch, part;
        if (tid < kDk) {
            ch = h * kDk + tid;
            part = 0;
        } else if (tid < 2 * kDk) {
            ch = kd + h * kDk + (tid - kDk);
            part = 1;
        } else {
            ch = 2 * kd + h * kDv + (tid - 2 * kDk);
            part = 2;
        }
        const float* w = d.conv_w + size_t(ch) * K;
        float* hist = d.conv_state + size_t(ch) * (K - 1);
        const float xv = d.projected[ch];
        float hv[8];
        float sum = 0.f;
        for (int i = 0; i < K - 1; ++i) {
            hv[i] = hist[i];
            sum += hv[i] * w[i];
        }
        sum += xv * w[K - 1];
        for (int i = 0; i + 1 < K - 1; ++i) hist[i] = hv[i + 1];
        if (K > 1) hist[K - 2] = xv;
        const float y = siluf_(sum);
        d.convolved[ch] = y;
        if (part == 0)
            qs[tid] = y;
        else if (part == 1)
            ks[tid - kDk] = y;
        else
            vs[tid - 2 * kDk] = y;
    }
    __syncthreads();
    // 2. L2 norms (the sums of squares over dk = 128 by threads 0..127)
    float sq = tid < kDk ? qs[tid] * qs[tid] : 0.f;
    float sk = tid < kDk ? ks[tid] * ks[tid] : 0.f;
    sq = block_sum(sq, red);
    sk = block_sum(sk, red);
    const float rq = 1.f / sqrtf(sq + 1e-6f), rk = 1.f / sqrtf(sk + 1e-6f), sd = sqrtf(float(kDk));
    __syncthreads();
    if (tid < kDk) {
        const float qn = (qs[tid] * rq) / sd, kn = ks[tid] * rk;
        qs[tid] = qn;
        ks[tid] = kn;
        d.query[size_t(h) * kDk + tid] = qn;
        d.key[size_t(h) * kDk + tid] = kn;
    }
    __syncthreads();
    // 3. gates (gates = [dt | A_log])
    const int vh = d.value_heads;
    const float log_decay = -expf(d.gates[vh + h]) * softplusf_(d.a[h] + d.gates[h]);
    const float beta = sigmoidf_(d.b[h]);
    const float decay = expf(log_decay);
    // 4. rule: lane = p * 16 + column-in-wave, 8 waves x 16 = 128 columns
    const int lane = tid & 63, wave = tid >> 6;
    const int p = lane / 16, j = wave * 16 + (lane % 16);
    float* state = d.recurrent + size_t(h) * kDk * kDv;
    float s[kKR];
#pragma unroll
    for (int ii = 0; ii < kKR; ++ii) s[ii] = state[size_t(p * kKR + ii) * kDv + j];
    float m = 0.f;
#pragma unroll
    for (int ii = 0; ii < kKR; ++ii) {
        s[ii] *= decay;
        m = fmaf(s[ii], ks[p * kKR + ii], m);
    }
    m += __shfl_xor(m, 16, 64);
    m += __shfl_xor(m, 32, 64);
    const float delta = (vs[j] - m) * beta;
    float out = 0.f;
#pragma unroll
    for (int ii = 0; ii < kKR; ++ii) {
        s[ii] = fmaf(ks[p * kKR + ii], delta, s[ii]);
        out = fmaf(s[ii], qs[p * kKR + ii], out);
    }
    out += __shfl_xor(out, 16, 64);
    out += __shfl_xor(out, 32, 64);
#pragma unroll
    for (int ii = 0; ii < kKR; ++ii) state[size_t(p * kKR + ii) * kDv + j] = s[ii];
    if (p == 0) {
        core[j] = out;
        d.core[size_t(h) * kDv + j] = out;
    }
    __syncthreads();
    // 5. gated RMSNorm (direct weight, offset 0)
    float ss = tid < kDv ? core[tid] * core[tid] : 0.f;
    ss = block_sum(ss, red);
    const float r = 1.f / sqrtf(ss / float(kDv) + d.eps);
    if (tid < kDv) {
        const size_t o = size_t(h) * kDv + tid;
        d.gated[o] = siluf_(d.z[o]) * ((core[tid] * r) * d.norm_w[tid]);
    }
}

}  // namespace

bool delta_mixer_decode_ok(const QrDelta& d) {
    return d.tokens == 1 && d.key_heads == d.value_heads && d.key_dim == kDk && d.value_dim == kDv &&
           d.kernel >= 1 && d.kernel <= 8 && d.channels == 2 * d.key_heads * kDk + d.value_heads * kDv;
}

int delta_mixer_decode(hipStream_t s, const QrDelta& d) {
    if (!delta_mixer_decode_ok(d)) return -1;
    hipLaunchKernelGGL(delta_mixer_decode_kernel, dim3(unsigned(d.value_heads)), dim3(kThreads), 0, s, d);
    return int(hipGetLastError());
}

}  // namespace qr
