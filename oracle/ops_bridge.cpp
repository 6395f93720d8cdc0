// TEST INFRASTRUCTURE ONLY. A CPU bridge exporting the qr_* ABI with
// qr_kind() == 0 (the reference's "CPU test bridge" kind, which the engine
// refuses outside tests): every op and projection computed by a scalar
// restatement of the reference's op bodies (native/rocm/reference.h:117-232,
// projections native/rocm/bridge.cpp:571-653). Tests use it to check the host
// engine's call sequence on the CPU and each HIP kernel op by op; it is pinned
// against the reference's own CPU test bridge (oracle/_ref, built from the
// reference's sources) op by op in tests/test_ops_bridge.py.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>

#include "../include/qwen_bridge.h"

struct Context {
    char error[256] = {};
    char info[64] = "CPU oracle op bridge (not HIP)";
};

namespace {

int fail(Context* c, const char* what) {
    std::snprintf(c->error, sizeof(c->error), "%s", what);
    return -1;
}
// reference.h:31-40
float sigmoid(float x) {
    if (x >= 0.f) return 1.f / (1.f + expf(-x));
    float e = expf(x);
    return e / (1.f + e);
}
float silu(float x) { return x * sigmoid(x); }
float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }
float bf16(uint16_t v) {
    uint32_t u = uint32_t(v) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
// reference.h:41-47: rotate-half over the first `dim` dims.
void rope(float* x, int dim, int pos, float theta) {
    for (int i = 0; i < dim / 2; ++i) {
        float angle = float(pos) / powf(theta, float(2 * i) / float(dim));
        float s = sinf(angle), c = cosf(angle), a = x[i], b = x[i + dim / 2];
        x[i] = a * c - b * s;
        x[i + dim / 2] = b * c + a * s;
    }
}
float inv_rms(const float* x, int d, float eps) {
    float sum = 0.f;
    for (int i = 0; i < d; ++i) sum += x[i] * x[i];
    return 1.f / sqrtf(sum / float(d) + eps);
}

// AttentionQuery item t (reference.h:75-84).
void attention_query(int t, const Params& a) {
    int d = a.n[0], rot = a.n[1], pos = a.n[2] + (a.n[3] > 0 ? t / a.n[3] : 0);
    const float* x = a.p[1] + size_t(t) * 2 * d;
    float r = inv_rms(x, d, a.f[0]);
    float* o = a.p[0] + size_t(t) * d;
    for (int i = 0; i < d; ++i) {
        o[i] = (x[i] * r) * (1.f + a.p[2][i]);
        a.p[3][size_t(t) * d + i] = x[d + i];
    }
    rope(o, rot, pos, a.f[1]);
}
// AttentionKv item t (reference.h:85-95).
void attention_kv(int t, const Params& a) {
    int d = a.n[0], rot = a.n[1], kv = a.n[3], pos = a.n[2] + t / kv, hh = t % kv;
    const float* x = a.p[1] + size_t(t) * d;
    float r = inv_rms(x, d, a.f[0]);
    size_t dest = (size_t(pos) * kv + hh) * d;
    for (int i = 0; i < d; ++i) {
        a.p[0][dest + i] = (x[i] * r) * (1.f + a.p[2][i]);
        a.p[4][dest + i] = a.p[3][size_t(t) * d + i];
    }
    rope(a.p[0] + dest, rot, pos, a.f[1]);
}

void op_body(int op, int t, const Params& a) {
    float *o = a.p[0], *x = a.p[1], *w = a.p[2];
    switch (op) {
    case QR_RMS_NORM: {
        int d = a.n[0];
        size_t off = size_t(t) * d;
        float r = inv_rms(x + off, d, a.f[0]);
        for (int i = 0; i < d; ++i) o[off + i] = (x[off + i] * r) * (w[i] + a.f[1]);
        break;
    }
    case QR_ADD: o[t] = x[t] + w[t]; break;
    case QR_SILU_PRODUCT: o[t] = silu(x[t]) * w[t]; break;
    case QR_CONV_SILU: {  // reference.h:96-116
        int k = a.n[0], tokens = a.n[1] > 0 ? a.n[1] : 1, stride = a.n[2];
        float* hist = a.p[3] + size_t(t) * (k - 1);
        for (int r = 0; r < tokens; ++r) {
            float xv = x[size_t(r) * stride + t], sum = 0.f;
            for (int i = 0; i < k - 1; ++i) sum += hist[i] * w[size_t(t) * k + i];
            sum += xv * w[size_t(t) * k + k - 1];
            for (int i = 0; i + 1 < k - 1; ++i) hist[i] = hist[i + 1];
            if (k > 1) hist[k - 2] = xv;
            o[size_t(r) * stride + t] = silu(sum);
            if (r < a.n[3])
                for (int i = 0; i < k - 1; ++i) hist[size_t(r + 1) * size_t(stride) * size_t(k - 1) + i] = hist[i];
        }
        break;
    }
    case QR_DELTA_QK: {  // reference.h:134-143
        int kh = a.n[0], vh = a.n[1], d = a.n[2], h = (t % vh) / (vh / kh), kd = kh * d;
        const float* xr = x + size_t(t / vh) * a.n[3];
        float sq = 0.f, sk = 0.f;
        for (int i = 0; i < d; ++i) {
            sq += xr[h * d + i] * xr[h * d + i];
            sk += xr[kd + h * d + i] * xr[kd + h * d + i];
        }
        float rq = 1.f / sqrtf(sq + 1e-6f), rk = 1.f / sqrtf(sk + 1e-6f);
        for (int i = 0; i < d; ++i) {
            o[size_t(t) * d + i] = (xr[h * d + i] * rq) / sqrtf(float(d));
            w[size_t(t) * d + i] = xr[kd + h * d + i] * rk;
        }
        break;
    }
    case QR_DELTA_GATES: {  // reference.h:144-148
        int head = a.n[0] > 0 ? t % a.n[0] : t;
        o[t] = -expf(a.p[4][head]) * softplus(x[t] + a.p[3][head]);
        a.p[5][t] = sigmoid(w[t]);
        break;
    }
    case QR_DELTA_RULE:
    case QR_DELTA_RULE_GATED: {  // reference.h:48-60, 149-170
        int kd = a.n[0], vd = a.n[1], kh = a.n[2], vh = a.n[3], h = t / vd, j = t % vd;
        int tokens = a.n[4] > 0 ? a.n[4] : 1, stride = a.n[5];
        float* state = a.p[4] + size_t(h) * kd * vd;
        for (int r = 0; r < tokens; ++r) {
            const float *q = x + size_t(r) * vh * kd, *k = w + size_t(r) * vh * kd, *v = a.p[3] + size_t(r) * stride;
            int i_gate = r * vh + h;
            float log_decay, beta;
            if (op == QR_DELTA_RULE_GATED) {
                log_decay = -expf(a.p[7][vh + h]) * softplus(a.p[5][i_gate] + a.p[7][h]);
                beta = sigmoid(a.p[6][i_gate]);
            } else {
                log_decay = a.p[5][i_gate];
                beta = a.p[6][i_gate];
            }
            float decay = expf(log_decay), memory = 0.f;
            for (int i = 0; i < kd; ++i) {
                state[size_t(i) * vd + j] *= decay;
                memory += state[size_t(i) * vd + j] * k[size_t(h) * kd + i];
            }
            float delta = (v[2 * size_t(kh) * kd + size_t(h) * vd + j] - memory) * beta, out = 0.f;
            for (int i = 0; i < kd; ++i) {
                state[size_t(i) * vd + j] += k[size_t(h) * kd + i] * delta;
                out += state[size_t(i) * vd + j] * q[size_t(h) * kd + i];
            }
            o[size_t(r) * vh * vd + t] = out;
            if (r < a.n[6])
                for (int i = 0; i < kd; ++i)
                    state[size_t(r + 1) * vh * kd * vd + size_t(i) * vd + j] = state[size_t(i) * vd + j];
        }
        break;
    }
    case QR_ATTENTION_QUERY: attention_query(t, a); break;
    case QR_ATTENTION_KV: attention_kv(t, a); break;
    case QR_ATTENTION_QUERY_KV: {  // reference.h:61-74: query items first, then KV items
        int queries = a.n[3] * a.n[5];
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
            attention_query(t, part);
        } else {
            part.p[0] = a.p[4];
            part.p[1] = a.p[5];
            part.p[2] = a.p[2] + a.n[0];
            part.p[3] = a.p[6];
            part.p[4] = a.p[7];
            part.n[3] = a.n[4];
            attention_kv(t - queries, part);
        }
        break;
    }
    case QR_ATTENTION_READ: {  // reference.h:173-193, score row of p5 per head
        int d = a.n[0], heads = a.n[1], kv = a.n[2], capacity = a.n[4], tokens = a.n[5] > 0 ? a.n[5] : 1;
        int h = t / (heads / kv);
        float* scores = a.p[5] + size_t(t) * capacity;
        for (int r = 0; r < tokens; ++r) {
            int length = a.n[3] + r;
            size_t row = (size_t(r) * heads + t) * d;
            float max = -INFINITY;
            for (int p = 0; p < length; ++p) {
                float sum = 0.f;
                for (int i = 0; i < d; ++i) sum += x[row + i] * w[(size_t(p) * kv + h) * d + i];
                scores[p] = sum / sqrtf(float(d));
                max = fmaxf(max, scores[p]);
            }
            float den = 0.f;
            for (int p = 0; p < length; ++p) {
                scores[p] = expf(scores[p] - max);
                den += scores[p];
            }
            for (int p = 0; p < length; ++p) scores[p] /= den;
            for (int i = 0; i < d; ++i) {
                float sum = 0.f;
                for (int p = 0; p < length; ++p) sum += scores[p] * a.p[3][(size_t(p) * kv + h) * d + i];
                o[row + i] = sum * sigmoid(a.p[4][row + i]);
            }
        }
        break;
    }
    case QR_EMBED_BF16: {
        const uint16_t* m = reinterpret_cast<const uint16_t*>(x);
        o[t] = bf16(m[size_t(a.n[0]) * size_t(a.n[1]) + size_t(t)]);
        break;
    }
    case QR_ADD_RMS_NORM: {  // reference.h:194-200
        int d = a.n[0];
        size_t off = size_t(t) * d;
        float sum = 0.f;
        for (int i = 0; i < d; ++i) {
            o[off + i] = a.p[1][off + i] + a.p[2][off + i];
            sum += o[off + i] * o[off + i];
        }
        float r = 1.f / sqrtf(sum / float(d) + a.f[0]);
        for (int i = 0; i < d; ++i) a.p[3][off + i] = (o[off + i] * r) * (a.p[4][i] + a.f[1]);
        break;
    }
    case QR_RMS_NORM_GATE: {  // reference.h:201-207
        int d = a.n[0];
        size_t off = size_t(t) * d;
        float r = inv_rms(x + off, d, a.f[0]);
        for (int i = 0; i < d; ++i) o[off + i] = silu(a.p[3][off + i]) * ((x[off + i] * r) * (w[i] + a.f[1]));
        break;
    }
    case QR_EMBED_BF16_PICKED: {  // reference.h:217-221
        const uint16_t* m = reinterpret_cast<const uint16_t*>(x);
        size_t h = size_t(a.n[1]), r = size_t(t) / h;
        o[t] = bf16(m[size_t(w[2 * r]) * h + size_t(t) % h]);
        break;
    }
    case QR_ARGMAX: {  // reference.h:222-230
        const float* v = x + size_t(t) * size_t(a.n[0]);
        float best = -INFINITY;
        unsigned at = 0xffffffffu, bad = 0;
        for (int i = 0; i < a.n[0]; ++i) {
            if (!std::isfinite(v[i])) {
                ++bad;
                continue;
            }
            if (v[i] > best) {
                best = v[i];
                at = unsigned(i);
            }
        }
        o[2 * t] = float(at);
        o[2 * t + 1] = float(bad);
        break;
    }
    }
}

enum class W { F32, BF16, I8 };
// Y[b, r] = sum_j A[r, j] X[b, j], one left-to-right sum per output
// (bridge.cpp:571-653 CPU branches; int8 scaled after the sum).
void project(W type, float* y, const float* a, const float* x, int rows, int cols, int batch) {
    for (int b = 0; b < batch; ++b)
        for (int i = 0; i < rows; ++i) {
            float sum = 0.f;
            for (int j = 0; j < cols; ++j) {
                size_t e = size_t(i) * cols + j;
                float wv = type == W::F32    ? a[e]
                           : type == W::BF16 ? bf16(reinterpret_cast<const uint16_t*>(a)[e])
                                             : float(reinterpret_cast<const int8_t*>(a + rows)[e]);
                sum += wv * x[size_t(b) * cols + j];
            }
            y[size_t(b) * rows + i] = type == W::I8 ? a[i] * sum : sum;
        }
}

}  // namespace

extern "C" {

int qr_abi(void) { return 3; }
int qr_kind(void) { return QR_KIND_CPU_TEST; }
int qr_max_op(void) { return QR_ATTENTION_QUERY_KV; }
int qr_snapshots(void) { return 1; }
int qr_argmax(void) { return 2; }
const char* qr_error(Context* c) { return c->error; }
const char* qr_info(Context* c) { return c->info; }
int qr_create(Context** out) {
    *out = new (std::nothrow) Context;
    return *out ? 0 : -1;
}
void qr_destroy(Context* c) { delete c; }
int qr_set_option(Context* c, const char* name, int value) {
    if (std::strcmp(name, "attention_f16") != 0 || (value != 0 && value != 1)) return fail(c, "unknown bridge option");
    return value ? fail(c, "attention_f16 needs a GPU bridge") : 0;
}
int qr_sync(Context*) { return 0; }
int qr_alloc(Context* c, float** p, size_t n) {
    *p = static_cast<float*>(std::calloc(n, sizeof(float)));
    return *p ? 0 : fail(c, "calloc");
}
void qr_free(Context*, float* p) { std::free(p); }
int qr_write(Context*, float* p, const float* host, size_t n) {
    std::memcpy(p, host, n * 4);
    return 0;
}
int qr_read(Context*, float* host, const float* p, size_t n) {
    std::memcpy(host, p, n * 4);
    return 0;
}
int qr_copy(Context*, float* dst, const float* src, size_t n) {
    std::memmove(dst, src, n * 4);
    return 0;
}
int qr_run(Context* c, int op, int count, const Params* a) {
    if (op < QR_RMS_NORM || op > QR_EMBED_BF16_PICKED || count < 1) return fail(c, "invalid kernel");
    if (op == QR_ARGMAX && a->n[0] < 1) return fail(c, "argmax shape");
    for (int t = 0; t < count; ++t) op_body(op, t, *a);
    return 0;
}
int qr_gemv(Context*, float* y, const float* a, const float* x, int rows, int cols) {
    project(W::F32, y, a, x, rows, cols, 1);
    return 0;
}
int qr_gemv_bf16(Context*, float* y, const float* a, const float* x, int rows, int cols) {
    project(W::BF16, y, a, x, rows, cols, 1);
    return 0;
}
int qr_gemm(Context* c, float* y, const float* a, const float* x, int rows, int cols, int batch) {
    if (rows < 1 || cols < 1 || batch < 1) return fail(c, "GEMM shape");
    project(W::F32, y, a, x, rows, cols, batch);
    return 0;
}
int qr_gemm_bf16(Context* c, float* y, const float* a, const float* x, int rows, int cols, int batch) {
    if (rows < 1 || cols < 1 || batch < 1) return fail(c, "bf16 GEMM shape");
    project(W::BF16, y, a, x, rows, cols, batch);
    return 0;
}
int qr_gemm_i8(Context* c, float* y, const float* a, const float* x, int rows, int cols, int batch) {
    if (rows < 1 || cols < 1 || batch < 1) return fail(c, "int8 GEMM shape");
    project(W::I8, y, a, x, rows, cols, batch);
    return 0;
}

}  // extern "C"
