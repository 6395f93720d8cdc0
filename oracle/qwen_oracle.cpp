// TEST INFRASTRUCTURE ONLY. CPU oracle: a restatement of the reference's Rust
// CPU forward pass (jl1nie/qwen-rust-inference), used by tests/, the smoke
// check and bench.py's cpu_baseline leg as the checker. The product (the HIP
// bridge and the host engine) never links, loads or calls this file.
//
// Every function names the reference file:line it follows. Arithmetic is f32
// with the reference's summation orders; built with -ffp-contract=off and
// without fast-math, so no multiply-add is contracted (Rust f32 semantics),
// and transcendental functions are glibc's expf/log1pf/powf/sinf/cosf, which is
// what Rust's f32::exp/ln_1p/powf/sin_cos lower to on Linux.
//
// Pinning (each checked in tests/test_oracle.py):
//   * whole model, every layer/op record: tests/golden/hybrid.json (official
//     PyTorch vectors) at the reference's 2e-5/2e-4, and
//     tests/golden/lesson-trace.ndjson (the reference's own Backend::Reference
//     outputs at f32 round-trip precision) at 2e-6/2e-5;
//   * chunked-prefill logits: hybrid.json "full_logits";
//   * rms_norm/silu/softmax/FFN: tests/golden/phase1.json;
//   * projections: integer-exact KATs and fp64 brute force;
//   * Vector backend vs Reference backend on every record (both reference
//     orders are restated; they differ only in summation order);
//   * int8 quantiser: the reference's invariants (|w - s q| <= s/2, zero row);
//   * attend: the reference's hand examples (tests/components.rs:117-150: the
//     1:3 read of 5 and the 4Q/2KV GQA grouping [3, 3, 12, 12]) and a float64
//     dense softmax at 8Q/2KV;
//   * rotate: the float64 closed form angle = pos * theta^(-2i/dim) at dims 8-64
//     and positions up to 8190;
//   * the whole forward on a config with 2 KV heads, rotary 16 of 32 and 2 key
//     heads for 4 value heads, bit for bit against the engine's op sequence on
//     the reference's own CPU test bridge (tests/test_engine_cpu.py).
#include "../include/qwen_model.h"

#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_error;

struct Fail {
    std::string what;
};
void require(bool ok, const char* what) {
    if (!ok) throw Fail{what};
}
// src/tensor.rs:33-36
void finite(const float* v, size_t n) {
    require(n > 0, "empty tensor");
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(v[i])) throw Fail{"NaN/Inf detected"};
}
void finite(const std::vector<float>& v) { finite(v.data(), v.size()); }

// Rust's `Iterator::sum` for f32 folds left from -0.0 (Rust 1.85, the
// reference's rust-toolchain.toml); only the sign of an all-zero sum differs
// from a fold from +0.0.
constexpr float kSumStart = -0.0f;

// ---------------------------------------------------------------- thread pool
// src/parallel.rs:40-91: output rows in contiguous blocks; each row is computed
// by one thread with the serial code, so results do not depend on the thread
// count. Threads = QWEN_THREADS or min(cores, 8); blocks need >= 2^15 work.
constexpr size_t kMinWorkPerBlock = size_t(1) << 15;

class Pool {
public:
    explicit Pool(int threads) : threads_(threads < 1 ? 1 : threads) {
        for (int i = 1; i < threads_; ++i) workers_.emplace_back([this] { work(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(m_);
            stop_ = true;
            ++generation_;
        }
        wake_.notify_all();
        for (auto& t : workers_) t.join();
    }
    int threads() const { return threads_; }
    // Runs task(0..blocks) on the workers and the calling thread.
    void run(size_t blocks, const std::function<void(size_t)>& task) {
        std::unique_lock<std::mutex> busy(exclusive_, std::try_to_lock);
        if (!busy.owns_lock() || threads_ == 1) {  // nested or concurrent: serial
            for (size_t i = 0; i < blocks; ++i) task(i);
            return;
        }
        {
            std::lock_guard<std::mutex> g(m_);
            task_ = &task;
            blocks_ = blocks;
            next_.store(0);
            active_ = int(workers_.size());
            ++generation_;
        }
        wake_.notify_all();
        claim(task, blocks);
        std::unique_lock<std::mutex> g(m_);
        done_.wait(g, [this] { return active_ == 0; });
        task_ = nullptr;
    }

private:
    void claim(const std::function<void(size_t)>& task, size_t blocks) {
        for (;;) {
            size_t i = next_.fetch_add(1);
            if (i >= blocks) return;
            task(i);
        }
    }
    void work() {
        uint64_t seen = 0;
        for (;;) {
            const std::function<void(size_t)>* task;
            size_t blocks;
            {
                std::unique_lock<std::mutex> g(m_);
                wake_.wait(g, [&] { return generation_ != seen; });
                seen = generation_;
                if (stop_) return;
                task = task_;
                blocks = blocks_;
            }
            if (task) claim(*task, blocks);
            std::lock_guard<std::mutex> g(m_);
            if (--active_ == 0) done_.notify_all();
        }
    }
    int threads_;
    std::vector<std::thread> workers_;
    std::mutex exclusive_, m_;
    std::condition_variable wake_, done_;
    const std::function<void(size_t)>* task_ = nullptr;
    size_t blocks_ = 0;
    std::atomic<size_t> next_{0};
    int active_ = 0;
    uint64_t generation_ = 0;
    bool stop_ = false;
};

int default_threads() {
    if (const char* e = std::getenv("QWEN_THREADS")) {
        int n = std::atoi(e);
        if (n > 0) return n;
    }
    unsigned hw = std::thread::hardware_concurrency();
    return int(hw == 0 ? 1 : (hw < 8 ? hw : 8));
}
Pool*& pool_slot() {
    static Pool* p = nullptr;
    return p;
}
Pool& pool() {
    Pool*& p = pool_slot();
    if (!p) p = new Pool(default_threads());
    return *p;
}

// src/parallel.rs:62-91
void for_blocks(size_t len, size_t work, const std::function<void(size_t, size_t)>& f) {
    size_t total = len * (work ? work : 1);
    size_t n = size_t(pool().threads());
    if (total / kMinWorkPerBlock < n) n = total / kMinWorkPerBlock;
    if (n < 1) n = 1;
    size_t block = (len + n - 1) / n;
    if (n <= 1 || block >= len) {
        f(0, len);
        return;
    }
    size_t blocks = (len + block - 1) / block;
    pool().run(blocks, [&](size_t i) {
        size_t first = i * block;
        size_t size = block < len - first ? block : len - first;
        f(first, size);
    });
}

// ---------------------------------------------------------------- projections
enum Backend { kReference = 0, kOptimized = 1, kVector = 2 };

// src/tensor.rs:325-331 (Reference): each row summed left to right from +0.0.
void linear_rows(const float* d, size_t cols, const float* x, float* out, size_t rows) {
    for (size_t r = 0; r < rows; ++r) {
        const float* row = d + r * cols;
        float y = 0.f;
        for (size_t j = 0; j < cols; ++j) y += row[j] * x[j];
        out[r] = y;
    }
}
// src/tensor.rs:338-352 (Vector, the inference default): eight interleaved
// partial sums over the whole chunks of 8, summed in lane order, then the tail.
void vector_rows(const float* d, size_t cols, const float* x, float* out, size_t rows) {
    size_t n = cols / 8 * 8;
    for (size_t r = 0; r < rows; ++r) {
        const float* row = d + r * cols;
        float sums[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (size_t j = 0; j < n; j += 8)
            for (int i = 0; i < 8; ++i) sums[i] += row[j + i] * x[j + i];
        float y = kSumStart;
        for (int i = 0; i < 8; ++i) y += sums[i];
        for (size_t j = n; j < cols; ++j) y += row[j] * x[j];
        out[r] = y;
    }
}

struct Matrix {
    const float* d = nullptr;
    size_t rows = 0, cols = 0;
};

// src/tensor.rs:244-254 (linear) and 279-296 (project).
std::vector<float> project(const Matrix& m, const std::vector<float>& x, int backend) {
    require(x.size() == m.cols, "linear input shape mismatch");
    require(backend == kReference || backend == kVector, "oracle backend must be Reference or Vector");
    finite(x);
    std::vector<float> out(m.rows, 0.f);
    for_blocks(m.rows, m.cols, [&](size_t first, size_t n) {
        if (backend == kReference)
            linear_rows(m.d + first * m.cols, m.cols, x.data(), out.data() + first, n);
        else
            vector_rows(m.d + first * m.cols, m.cols, x.data(), out.data() + first, n);
    });
    finite(out);
    return out;
}

// ---------------------------------------------------------------- elementwise
// src/ops.rs:71-78
float sigmoid(float x) {
    if (x >= 0.f) return 1.f / (1.f + expf(-x));
    float e = expf(x);
    return e / (1.f + e);
}
// src/ops.rs:16-32
std::vector<float> silu(const std::vector<float>& x) {
    finite(x);
    std::vector<float> out(x.size());
    for (size_t i = 0; i < x.size(); ++i) out[i] = x[i] * sigmoid(x[i]);
    finite(out);
    return out;
}
// src/ops.rs:1-15 (binary add / multiply)
std::vector<float> add(const std::vector<float>& a, const std::vector<float>& b) {
    require(a.size() == b.size(), "elementwise shape mismatch");
    std::vector<float> out(a.size());
    for (size_t i = 0; i < a.size(); ++i) out[i] = a[i] + b[i];
    finite(out);
    return out;
}
std::vector<float> multiply(const std::vector<float>& a, const std::vector<float>& b) {
    require(a.size() == b.size(), "elementwise shape mismatch");
    std::vector<float> out(a.size());
    for (size_t i = 0; i < a.size(); ++i) out[i] = a[i] * b[i];
    finite(out);
    return out;
}
// src/ops.rs:33-42
std::vector<float> softmax(const std::vector<float>& x) {
    finite(x);
    float max = -INFINITY;
    for (float v : x) max = std::fmax(max, v);
    std::vector<float> e(x.size());
    float sum = kSumStart;
    for (size_t i = 0; i < x.size(); ++i) {
        e[i] = expf(x[i] - max);
    }
    for (float v : e) sum += v;
    require(std::isfinite(sum) && sum > 0.f, "invalid softmax denominator");
    for (auto& v : e) v = v / sum;
    finite(e);
    return e;
}
// src/ops.rs:48-70: Direct multiplies by w, QwenZeroCentered by (1 + w).
std::vector<float> rms_norm(const float* x, size_t n, const float* w, float eps, bool zero_centered) {
    finite(x, n);
    finite(w, n);
    float ss = kSumStart;
    for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float mean = ss / float(n);
    float denominator = mean + eps;
    require(std::isfinite(denominator), "RMSNorm variance overflow");
    float inverse = 1.f / std::sqrt(denominator);
    std::vector<float> out(n);
    for (size_t i = 0; i < n; ++i) {
        float s = zero_centered ? 1.f + w[i] : w[i];
        out[i] = (x[i] * inverse) * s;
    }
    finite(out);
    return out;
}
// src/ops.rs:79-85
float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }
// src/ops.rs:86-92
std::vector<float> l2_norm(const float* x, size_t n) {
    finite(x, n);
    float s = kSumStart;
    for (size_t i = 0; i < n; ++i) s += x[i] * x[i];
    s = s + 1e-6f;
    require(std::isfinite(s), "L2 variance overflow");
    float r = 1.f / std::sqrt(s);
    std::vector<float> out(n);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * r;
    return out;
}
// src/attention.rs:41-57: rotate-half over the first `dim` dims.
void rotate(float* x, size_t len, size_t position, size_t dim, float theta) {
    require(dim <= len && dim % 2 == 0 && std::isfinite(theta) && theta > 0.f, "invalid RoPE");
    for (size_t i = 0; i < dim / 2; ++i) {
        float angle = float(position) / powf(theta, float(2 * i) / float(dim));
        float s = sinf(angle), c = cosf(angle);
        float a = x[i], b = x[i + dim / 2];
        x[i] = a * c - b * s;
        x[i + dim / 2] = b * c + a * s;
    }
    finite(x, len);
}

}  // namespace

// ---------------------------------------------------------------- model
typedef void (*qo_trace_fn)(void* user, int layer, const char* name, const float* values, int64_t n);

struct qo_model {
    QwConfig c{};
    Matrix embedding;
    Matrix lm_head;  // the vocabulary projection; the embedding unless replaced
    const float* norm = nullptr;
    struct Layer {
        bool attention = false;
        const float *input_norm, *post_norm;
        Matrix gate, up, down;
        // attention
        Matrix q, k, v, o;
        const float *q_norm, *k_norm;
        // delta
        Matrix qkv, z, a, b, out;
        const float *conv, *dt, *a_log, *dnorm;
    };
    std::vector<Layer> layers;
    struct Edit {
        size_t layer;
        std::vector<size_t> columns;
        std::vector<float> direction;  // empty: disable the units
        float coefficient;
    };
    std::vector<Edit> edits;  // the EditManifest applied by every step (src/edit.rs)
    size_t channels() const { return size_t(2 * c.key_heads * c.key_dim + c.value_heads * c.value_dim); }
};

struct qo_state {
    size_t position = 0;
    struct Layer {
        std::vector<std::vector<float>> keys, values;  // KvCache (src/state.rs:4-8)
        std::vector<float> conv, recurrent;             // DeltaState (src/state.rs:9-14)
    };
    std::vector<Layer> layers;
};

namespace {

struct Tracer {
    qo_trace_fn fn;
    void* user;
    void operator()(int layer, const char* name, const std::vector<float>& v) const {
        if (fn) fn(user, layer, name, v.data(), int64_t(v.size()));
    }
};

// src/attention.rs:72-130 (attend_traced): per query head h the KV head
// h / (heads / kv_heads) (contiguous groups), scores q.k / sqrt(d) over every
// cached position, softmax, probability-weighted sum of the values.
std::vector<float> attend(const float* query, const std::vector<std::vector<float>>& keys,
                          const std::vector<std::vector<float>>& values, size_t heads, size_t kvh, size_t d,
                          std::vector<float>* all_scores, std::vector<float>* all_probs) {
    require(heads > 0 && kvh > 0 && d > 0 && heads % kvh == 0, "invalid GQA");
    require(!keys.empty() && keys.size() == values.size(), "attention shape mismatch");
    finite(query, heads * d);
    for (size_t p = 0; p < keys.size(); ++p) {
        require(keys[p].size() == kvh * d && values[p].size() == kvh * d, "KV shape mismatch");
        finite(keys[p]);
        finite(values[p]);
    }
    std::vector<float> out(heads * d, 0.f);
    for (size_t h = 0; h < heads; ++h) {
        size_t kv = h / (heads / kvh);
        const float* q = query + h * d;
        std::vector<float> scores(keys.size());
        for (size_t p = 0; p < keys.size(); ++p) {
            const float* kk = keys[p].data() + kv * d;
            float sum = kSumStart;
            for (size_t i = 0; i < d; ++i) sum += q[i] * kk[i];
            scores[p] = sum / std::sqrt(float(d));
        }
        auto probs = softmax(scores);
        if (all_scores) all_scores->insert(all_scores->end(), scores.begin(), scores.end());
        if (all_probs) all_probs->insert(all_probs->end(), probs.begin(), probs.end());
        for (size_t p = 0; p < values.size(); ++p)
            for (size_t i = 0; i < d; ++i) out[h * d + i] += probs[p] * values[p][kv * d + i];
    }
    finite(out);
    return out;
}

// src/attention.rs:132-226 (project, step) and 189-207 (finish).
std::vector<float> attention_step(const qo_model& m, const qo_model::Layer& w, const std::vector<float>& x,
                                  qo_state::Layer& s, size_t position, int backend, int layer, const Tracer& tr) {
    const QwConfig& c = m.c;
    size_t d = size_t(c.head_dim), heads = size_t(c.num_heads), kvh = size_t(c.num_kv_heads);
    require(position == s.keys.size() && s.values.size() == position, "KV position mismatch");
    // project (src/attention.rs:132-188)
    std::vector<float> mixed = project(w.q, x, backend);
    std::vector<float> key = project(w.k, x, backend);
    std::vector<float> value = project(w.v, x, backend);
    require(mixed.size() == heads * d * 2 && key.size() == kvh * d && value.size() == key.size(),
            "attention projection shape");
    std::vector<float> query, gate;
    for (size_t h = 0; h < heads; ++h) {
        const float* head = mixed.data() + h * 2 * d;
        auto q = rms_norm(head, d, w.q_norm, c.rms_norm_eps, true);
        query.insert(query.end(), q.begin(), q.end());
        gate.insert(gate.end(), head + d, head + 2 * d);
    }
    std::vector<float> projected_key = key;
    std::vector<float> query_before_rope = query;
    for (size_t h = 0; h < heads; ++h) rotate(query.data() + h * d, d, position, size_t(c.rotary_dim), c.rope_theta);
    for (size_t h = 0; h < kvh; ++h) {
        auto kn = rms_norm(key.data() + h * d, d, w.k_norm, c.rms_norm_eps, true);
        std::memcpy(key.data() + h * d, kn.data(), d * sizeof(float));
    }
    std::vector<float> key_before_rope = key;
    for (size_t h = 0; h < kvh; ++h) rotate(key.data() + h * d, d, position, size_t(c.rotary_dim), c.rope_theta);
    // step: the cache keeps the rotated key and the raw value (src/attention.rs:208-226)
    s.keys.push_back(key);
    s.values.push_back(value);
    std::vector<float> all_scores, all_probs;
    std::vector<float> out = attend(query.data(), s.keys, s.values, heads, kvh, d, &all_scores, &all_probs);
    std::vector<float> gated = out;
    for (size_t i = 0; i < gated.size(); ++i) gated[i] *= sigmoid(gate[i]);
    std::vector<float> output = project(w.o, gated, backend);
    tr(layer, "attention.projected_q_gate", mixed);
    tr(layer, "attention.projected_k", projected_key);
    tr(layer, "attention.q_before_rope", query_before_rope);
    tr(layer, "attention.k_before_rope", key_before_rope);
    tr(layer, "attention.q", query);
    tr(layer, "attention.k", key);
    tr(layer, "attention.v", value);
    tr(layer, "attention.gate", gate);
    tr(layer, "attention.scores", all_scores);
    tr(layer, "attention.probabilities", all_probs);
    tr(layer, "attention.context", out);
    tr(layer, "attention.gated", gated);
    return output;
}

// src/deltanet.rs:48-100: one head, state row-major [key_dim, value_dim].
std::vector<float> delta_rule(const float* q, const float* k, const float* v, size_t kd, size_t vd, float g,
                              float beta, float* state) {
    finite(q, kd);
    finite(k, kd);
    finite(v, vd);
    finite(state, kd * vd);
    require(std::isfinite(g) && g <= 0.f && std::isfinite(beta) && beta >= 0.f && beta <= 1.f,
            "invalid delta rule input");
    float decay = expf(g);
    for (size_t i = 0; i < kd * vd; ++i) state[i] *= decay;
    std::vector<float> delta(v, v + vd);
    for (size_t j = 0; j < vd; ++j) {
        float memory = kSumStart;
        for (size_t i = 0; i < kd; ++i) memory += state[i * vd + j] * k[i];
        delta[j] = (delta[j] - memory) * beta;
    }
    for (size_t i = 0; i < kd; ++i)
        for (size_t j = 0; j < vd; ++j) state[i * vd + j] += k[i] * delta[j];
    std::vector<float> out(vd);
    for (size_t j = 0; j < vd; ++j) {
        float sum = kSumStart;
        for (size_t i = 0; i < kd; ++i) sum += state[i * vd + j] * q[i];
        out[j] = sum;
    }
    finite(state, kd * vd);
    finite(out);
    return out;
}

// src/deltanet.rs:117-248 (step_captured).
std::vector<float> delta_step(const qo_model& m, const qo_model::Layer& w, const std::vector<float>& x,
                              qo_state::Layer& s, int backend, int layer, const Tracer& tr) {
    const QwConfig& c = m.c;
    size_t channels = w.qkv.rows, K = size_t(c.conv_kernel);
    size_t kh = size_t(c.key_heads), vh = size_t(c.value_heads), dk = size_t(c.key_dim), dv = size_t(c.value_dim);
    require(K > 0 && kh > 0 && vh % kh == 0 && dk > 0 && dv > 0, "invalid DeltaNet config");
    require(s.conv.size() == channels * (K - 1) && s.recurrent.size() == vh * dk * dv, "DeltaNet state shape mismatch");
    std::vector<float> projected = project(w.qkv, x, backend);
    std::vector<float> convolved(channels, 0.f);
    for (size_t ch = 0; ch < channels; ++ch) {
        const float* weights = w.conv + ch * K;
        float* history = s.conv.data() + ch * (K - 1);
        float sum = 0.f;
        for (size_t i = 0; i < K - 1; ++i) sum += history[i] * weights[i];
        sum += projected[ch] * weights[K - 1];
        convolved[ch] = sum;
        if (K > 1) {
            for (size_t i = 0; i + 1 < K - 1; ++i) history[i] = history[i + 1];
            history[K - 2] = projected[ch];
        }
    }
    std::vector<float> convolution_sums = convolved;
    convolved = silu(convolved);
    size_t kd = kh * dk, vd = vh * dv;
    require(convolved.size() == 2 * kd + vd, "DeltaNet QKV shape");
    std::vector<float> query, key, value(convolved.begin() + long(2 * kd), convolved.end());
    for (size_t h = 0; h < vh; ++h) {
        size_t k_head = h / (vh / kh);
        auto q = l2_norm(convolved.data() + k_head * dk, dk);
        auto k = l2_norm(convolved.data() + kd + k_head * dk, dk);
        query.insert(query.end(), q.begin(), q.end());
        key.insert(key.end(), k.begin(), k.end());
    }
    for (auto& q : query) q /= std::sqrt(float(dk));
    std::vector<float> a = project(w.a, x, backend);
    std::vector<float> b = project(w.b, x, backend);
    std::vector<float> z = project(w.z, x, backend);
    require(a.size() == vh && b.size() == vh, "DeltaNet gate shape");
    std::vector<float> beta(vh), decay(vh);
    for (size_t h = 0; h < vh; ++h) {
        beta[h] = sigmoid(b[h]);
        decay[h] = -expf(w.a_log[h]) * softplus(a[h] + w.dt[h]);
    }
    std::vector<float> core;
    for (size_t h = 0; h < vh; ++h) {
        auto o = delta_rule(query.data() + h * dk, key.data() + h * dk, value.data() + h * dv, dk, dv, decay[h],
                            beta[h], s.recurrent.data() + h * dk * dv);
        core.insert(core.end(), o.begin(), o.end());
    }
    require(z.size() == core.size(), "DeltaNet output gate shape");
    std::vector<float> gated;
    for (size_t h = 0; h < vh; ++h) {
        auto n = rms_norm(core.data() + h * dv, dv, w.dnorm, c.rms_norm_eps, false);
        std::vector<float> zh(z.begin() + long(h * dv), z.begin() + long((h + 1) * dv));
        auto g = multiply(n, silu(zh));
        gated.insert(gated.end(), g.begin(), g.end());
    }
    std::vector<float> output = project(w.out, gated, backend);
    tr(layer, "delta.projected", projected);
    tr(layer, "delta.conv_sum", convolution_sums);
    tr(layer, "delta.a", a);
    tr(layer, "delta.b", b);
    tr(layer, "delta.z", z);
    tr(layer, "delta.conv_silu", convolved);
    tr(layer, "delta.q", query);
    tr(layer, "delta.k", key);
    tr(layer, "delta.v", value);
    tr(layer, "delta.decay_log", decay);
    tr(layer, "delta.beta", beta);
    tr(layer, "delta.core", core);
    tr(layer, "delta.gated", gated);
    if (tr.fn) {
        tr(layer, "delta.recurrent_state", s.recurrent);
        if (!s.conv.empty()) tr(layer, "delta.conv_state", s.conv);
    }
    return output;
}

// EditManifest::apply (src/edit.rs:59-110): direction-less edits scale their
// product units by (1 - coefficient); then each direction edit adds
// -coefficient * d * (d . w_j) / (d . d) * product[j] for its columns j
// (w_j = column j of down), every sum a left fold.
std::vector<float> apply_edits(const qo_model& m, size_t layer, std::vector<float>& product, const Matrix& down) {
    require(product.size() == down.cols, "edit product shape mismatch");
    std::vector<float> correction(down.rows, 0.f);
    for (const auto& e : m.edits)
        if (e.layer == layer && e.direction.empty())
            for (size_t j : e.columns) product[j] *= 1.f - e.coefficient;
    for (const auto& e : m.edits) {
        if (e.layer != layer || e.direction.empty()) continue;
        float denominator = kSumStart;
        for (float v : e.direction) denominator += v * v;
        for (size_t j : e.columns) {
            float dot = kSumStart;
            for (size_t r = 0; r < down.rows; ++r) dot += e.direction[r] * down.d[r * down.cols + j];
            const float projection = dot / denominator;
            for (size_t r = 0; r < down.rows; ++r) correction[r] -= e.coefficient * e.direction[r] * projection * product[j];
        }
    }
    finite(correction);
    return correction;
}

// src/model.rs:53-99 (step_hidden) with src/block.rs:55-101 and src/ffn.rs:41-75.
void model_step(const qo_model& m, qo_state& st, uint32_t id, int backend, float* logits_out, float* norm_out,
                const Tracer& tr) {
    const QwConfig& c = m.c;
    size_t H = size_t(c.hidden_size);
    require(st.layers.size() == m.layers.size() && st.position < size_t(c.max_positions),
            "model state/context mismatch");
    require(id < uint32_t(c.vocab_size), "row out of bounds");
    std::vector<float> x(m.embedding.d + size_t(id) * H, m.embedding.d + size_t(id + 1) * H);
    tr(0, "embedding", x);
    for (size_t l = 0; l < m.layers.size(); ++l) {
        const auto& w = m.layers[l];
        int L = int(l);
        tr(L, "input", x);
        auto input_norm = rms_norm(x.data(), H, w.input_norm, c.rms_norm_eps, true);
        tr(L, "input_norm", input_norm);
        std::vector<float> mixed = w.attention
                                       ? attention_step(m, w, input_norm, st.layers[l], st.position, backend, L, tr)
                                       : delta_step(m, w, input_norm, st.layers[l], backend, L, tr);
        auto after_mixer = add(x, mixed);
        auto post_norm = rms_norm(after_mixer.data(), H, w.post_norm, c.rms_norm_eps, true);
        // FFN (src/ffn.rs:41-75) with the edit manifest (src/edit.rs:59-110)
        auto gate = project(w.gate, post_norm, backend);
        auto up = project(w.up, post_norm, backend);
        auto activated = silu(gate);
        auto product = multiply(activated, up);
        auto intervened = product;
        auto correction = apply_edits(m, l, intervened, w.down);
        auto down = project(w.down, intervened, backend);
        auto ffn = add(down, correction);
        auto output = add(after_mixer, ffn);
        tr(L, "mixer", mixed);
        tr(L, "after_mixer", after_mixer);
        tr(L, "post_norm", post_norm);
        tr(L, "ffn.gate", gate);
        tr(L, "ffn.up", up);
        tr(L, "ffn.silu", activated);
        tr(L, "ffn.product", product);
        tr(L, "ffn.intervened_product", intervened);
        tr(L, "ffn.output", ffn);
        tr(L, "layer", output);
        x = std::move(output);
    }
    auto normalized = rms_norm(x.data(), H, m.norm, c.rms_norm_eps, true);
    auto logits = project(m.lm_head, normalized, backend);
    int last = int(m.layers.size()) - 1;
    tr(last, "final_norm", normalized);
    tr(last, "logits", logits);
    if (logits_out) std::memcpy(logits_out, logits.data(), logits.size() * sizeof(float));
    if (norm_out) std::memcpy(norm_out, normalized.data(), H * sizeof(float));
    st.position += 1;
}

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const Fail& e) {
        g_error = e.what;
    } catch (const std::exception& e) {
        g_error = e.what();
    }
    return -1;
}

}  // namespace

extern "C" {

const char* qo_error() { return g_error.c_str(); }

int qo_set_threads(int n) {
    return guarded([&] {
        Pool*& p = pool_slot();
        delete p;
        p = new Pool(n > 0 ? n : default_threads());
    });
}
int qo_threads() { return pool().threads(); }

// `tensors` follows the slot order of include/qwen_model.h. The arrays are
// borrowed: they must outlive the model.
qo_model* qo_model_create(const QwConfig* cfg, const float* const* tensors) {
    qo_model* m = nullptr;
    int s = guarded([&] {
        const QwConfig& c = *cfg;
        require(c.hidden_size > 0 && c.intermediate_size > 0 && c.vocab_size > 0 && c.num_layers > 0 &&
                    c.num_layers <= QW_MAX_LAYERS && c.max_positions > 0,
                "zero config dimension");
        require(c.num_kv_heads > 0 && c.num_heads > 0 && c.num_heads % c.num_kv_heads == 0 && c.head_dim > 0,
                "invalid attention heads");
        require(c.key_heads > 0 && c.value_heads > 0 && c.value_heads % c.key_heads == 0 && c.key_dim > 0 &&
                    c.value_dim > 0 && c.conv_kernel > 0,
                "invalid DeltaNet dimensions");
        require(c.rotary_dim > 0 && c.rotary_dim % 2 == 0 && c.rotary_dim <= c.head_dim, "unsupported RoPE");
        auto* mm = new qo_model;
        mm->c = c;
        size_t H = size_t(c.hidden_size), I = size_t(c.intermediate_size);
        mm->embedding = Matrix{tensors[0], size_t(c.vocab_size), H};
        mm->lm_head = mm->embedding;
        mm->norm = tensors[1];
        size_t ch = mm->channels();
        for (int l = 0; l < c.num_layers; ++l) {
            const float* const* t = tensors + QW_SLOTS_BASE + size_t(l) * QW_SLOTS_LAYER;
            qo_model::Layer w{};
            w.attention = c.attention[l] != 0;
            w.input_norm = t[QW_INPUT_NORM];
            w.post_norm = t[QW_POST_NORM];
            w.gate = Matrix{t[QW_GATE], I, H};
            w.up = Matrix{t[QW_UP], I, H};
            w.down = Matrix{t[QW_DOWN], H, I};
            if (w.attention) {
                size_t d = size_t(c.head_dim), q = size_t(c.num_heads) * d, kv = size_t(c.num_kv_heads) * d;
                w.q = Matrix{t[QW_Q], 2 * q, H};
                w.k = Matrix{t[QW_K], kv, H};
                w.v = Matrix{t[QW_V], kv, H};
                w.o = Matrix{t[QW_O], H, q};
                w.q_norm = t[QW_Q_NORM];
                w.k_norm = t[QW_K_NORM];
            } else {
                size_t vd = size_t(c.value_heads) * size_t(c.value_dim), vh = size_t(c.value_heads);
                w.qkv = Matrix{t[QW_QKV], ch, H};
                w.z = Matrix{t[QW_Z], vd, H};
                w.a = Matrix{t[QW_A], vh, H};
                w.b = Matrix{t[QW_B], vh, H};
                w.conv = t[QW_CONV];
                w.dt = t[QW_DT];
                w.a_log = t[QW_A_LOG];
                w.dnorm = t[QW_DELTA_NORM];
                w.out = Matrix{t[QW_OUT], H, vd};
            }
            mm->layers.push_back(w);
        }
        m = mm;
    });
    return s == 0 ? m : nullptr;
}
void qo_model_free(qo_model* m) { delete m; }

// A separate vocabulary projection [vocab, hidden] (borrowed): the int8
// format projects with its own copy while the lookup keeps the embedding
// rows (reference src/device.rs:987-996).
void qo_model_set_lm_head(qo_model* m, const float* w) { m->lm_head.d = w ? w : m->embedding.d; }

// src/model.rs:322-334 (new_state): empty KV, zero DeltaNet state.
qo_state* qo_state_create(const qo_model* m) {
    auto* s = new qo_state;
    s->layers.resize(m->layers.size());
    for (size_t l = 0; l < m->layers.size(); ++l)
        if (!m->layers[l].attention) {
            s->layers[l].conv.assign(m->channels() * size_t(m->c.conv_kernel - 1), 0.f);
            s->layers[l].recurrent.assign(
                size_t(m->c.value_heads) * size_t(m->c.key_dim) * size_t(m->c.value_dim), 0.f);
        }
    return s;
}
qo_state* qo_state_clone(const qo_state* s) { return new qo_state(*s); }
void qo_state_free(qo_state* s) { delete s; }
int64_t qo_state_position(const qo_state* s) { return int64_t(s->position); }

// Size in floats of one state part: which = 0 conv history, 1 recurrent,
// 2 keys (position * kv * d), 3 values.
int64_t qo_state_size(const qo_model* m, const qo_state* s, int layer, int which) {
    if (layer < 0 || size_t(layer) >= s->layers.size()) return -1;
    const auto& L = s->layers[size_t(layer)];
    bool att = m->layers[size_t(layer)].attention;
    switch (which) {
    case 0: return att ? 0 : int64_t(L.conv.size());
    case 1: return att ? 0 : int64_t(L.recurrent.size());
    case 2: return att ? int64_t(L.keys.size()) * m->c.num_kv_heads * m->c.head_dim : 0;
    case 3: return att ? int64_t(L.values.size()) * m->c.num_kv_heads * m->c.head_dim : 0;
    }
    return -1;
}
int qo_state_read(const qo_model* m, const qo_state* s, int layer, int which, float* out) {
    int64_t n = qo_state_size(m, s, layer, which);
    if (n < 0) {
        g_error = "state part";
        return -1;
    }
    const auto& L = s->layers[size_t(layer)];
    switch (which) {
    case 0: std::memcpy(out, L.conv.data(), size_t(n) * 4); break;
    case 1: std::memcpy(out, L.recurrent.data(), size_t(n) * 4); break;
    case 2:
    case 3: {
        const auto& rows = which == 2 ? L.keys : L.values;
        size_t w = size_t(m->c.num_kv_heads * m->c.head_dim);
        for (size_t p = 0; p < rows.size(); ++p) std::memcpy(out + p * w, rows[p].data(), w * 4);
        break;
    }
    }
    return 0;
}
// Replaces the whole state with `position` tokens' worth (the reference's
// load_state for a CPU ModelState, src/device.rs:2380-2537): parts[layer * 4 +
// which] as qo_state_read lays them out (keys / values: position rows).
int qo_state_load(const qo_model* m, qo_state* s, int64_t position, const float* const* parts) {
    return guarded([&] {
        require(position >= 0, "state position");
        size_t w = size_t(m->c.num_kv_heads * m->c.head_dim);
        for (size_t l = 0; l < s->layers.size(); ++l) {
            auto& L = s->layers[l];
            const float* const* p = parts + 4 * l;
            if (m->layers[l].attention) {
                require(position == 0 || (p[2] && p[3]), "state part missing");
                L.keys.assign(size_t(position), std::vector<float>(w));
                L.values.assign(size_t(position), std::vector<float>(w));
                for (size_t r = 0; r < size_t(position); ++r) {
                    std::memcpy(L.keys[r].data(), p[2] + r * w, w * 4);
                    std::memcpy(L.values[r].data(), p[3] + r * w, w * 4);
                }
            } else {
                require(p[0] && p[1], "state part missing");
                std::memcpy(L.conv.data(), p[0], L.conv.size() * 4);
                std::memcpy(L.recurrent.data(), p[1], L.recurrent.size() * 4);
            }
        }
        s->position = size_t(position);
    });
}

// One token through the model (Model::step, src/model.rs:335-382). backend:
// 0 = Backend::Reference, 2 = Backend::Vector. logits_out: vocab floats (or
// NULL); norm_out: hidden floats of the final norm (or NULL). `trace` (may be
// NULL) receives every record of src/trace.rs:117-222 by name.
int qo_step(const qo_model* m, qo_state* s, uint32_t id, int backend, float* logits_out, float* norm_out,
            qo_trace_fn trace, void* user) {
    return guarded([&] { model_step(*m, *s, id, backend, logits_out, norm_out, Tracer{trace, user}); });
}

// Greedy selection (src/generate.rs:30-41): the first index of the maximum;
// non-finite logits are an error.
int64_t qo_select_greedy(const float* logits, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        if (!std::isfinite(logits[i])) {
            g_error = "NaN/Inf detected";
            return -1;
        }
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i)
        if (logits[i] > logits[best]) best = i;
    return best;
}

// Row-wise symmetric int8 quantiser (src/device.rs:220-239): scale = max|w| /
// 127, q = round-half-even(w / scale) clamped to +-127; a zero row has scale 0.
void qo_quantize_int8_rows(const float* w, int64_t rows, int64_t cols, float* scales, int8_t* q) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = w + r * cols;
        float max = 0.f;
        for (int64_t j = 0; j < cols; ++j) max = std::fmax(max, std::fabs(row[j]));
        float scale = max / 127.f;
        scales[r] = scale;
        for (int64_t j = 0; j < cols; ++j) {
            if (scale == 0.f) {
                q[r * cols + j] = 0;
                continue;
            }
            float v = std::nearbyint(row[j] / scale);  // default rounding mode: ties to even
            v = std::fmin(127.f, std::fmax(-127.f, v));
            q[r * cols + j] = int8_t(v);
        }
    }
}

// The reference's Matrix::project on one input vector (backend 0 Reference,
// 2 Vector), for projection KATs.
int qo_project(const float* w, int64_t rows, int64_t cols, const float* x, int backend, float* out) {
    return guarded([&] {
        Matrix m{w, size_t(rows), size_t(cols)};
        std::vector<float> xv(x, x + cols);
        auto y = project(m, xv, backend);
        std::memcpy(out, y.data(), y.size() * 4);
    });
}
int qo_rms_norm(const float* x, int64_t n, const float* w, float eps, int zero_centered, float* out) {
    return guarded([&] {
        auto y = rms_norm(x, size_t(n), w, eps, zero_centered != 0);
        std::memcpy(out, y.data(), y.size() * 4);
    });
}
int qo_softmax(const float* x, int64_t n, float* out) {
    return guarded([&] {
        auto y = softmax(std::vector<float>(x, x + n));
        std::memcpy(out, y.data(), y.size() * 4);
    });
}
int qo_silu(const float* x, int64_t n, float* out) {
    return guarded([&] {
        auto y = silu(std::vector<float>(x, x + n));
        std::memcpy(out, y.data(), y.size() * 4);
    });
}
int qo_delta_rule(const float* q, const float* k, const float* v, int64_t kd, int64_t vd, float g, float beta,
                  float* state, float* out) {
    return guarded([&] {
        auto y = delta_rule(q, k, v, size_t(kd), size_t(vd), g, beta, state);
        std::memcpy(out, y.data(), y.size() * 4);
    });
}
// The edit manifest every following step applies (Model::step's edit,
// src/model.rs:53-99): n edits; edit k has layer layers[k], columns
// columns[offsets[k] .. offsets[k + 1]), direction directions[k] (hidden
// floats, or NULL) and coefficients[k]. n = 0 removes it.
int qo_model_set_edit(qo_model* m, int64_t n, const int32_t* layers, const int64_t* offsets, const int64_t* columns,
                      const float* const* directions, const float* coefficients) {
    return guarded([&] {
        std::vector<qo_model::Edit> out;
        for (int64_t k = 0; k < n; ++k) {
            require(layers[k] >= 0 && size_t(layers[k]) < m->layers.size(), "edit target mismatch");
            qo_model::Edit e;
            e.layer = size_t(layers[k]);
            for (int64_t j = offsets[k]; j < offsets[k + 1]; ++j) {
                require(columns[j] >= 0 && columns[j] < m->c.intermediate_size, "invalid edit target");
                e.columns.push_back(size_t(columns[j]));
            }
            if (directions && directions[k])
                e.direction.assign(directions[k], directions[k] + m->c.hidden_size);
            e.coefficient = coefficients[k];
            out.push_back(std::move(e));
        }
        m->edits = std::move(out);
    });
}
// attend (src/attention.rs:63-71): query [heads * d]; keys / values [positions][kv_heads * d].
int qo_attend(const float* query, const float* keys, const float* values, int64_t positions, int64_t heads,
              int64_t kv_heads, int64_t d, float* out) {
    return guarded([&] {
        require(positions > 0 && kv_heads > 0 && d > 0, "invalid attention shape");
        size_t row = size_t(kv_heads * d);
        std::vector<std::vector<float>> k, v;
        for (int64_t p = 0; p < positions; ++p) {
            k.emplace_back(keys + size_t(p) * row, keys + size_t(p + 1) * row);
            v.emplace_back(values + size_t(p) * row, values + size_t(p + 1) * row);
        }
        auto o = attend(query, k, v, size_t(heads), size_t(kv_heads), size_t(d), nullptr, nullptr);
        std::memcpy(out, o.data(), o.size() * sizeof(float));
    });
}
int qo_rotate(float* x, int64_t len, int64_t position, int64_t dim, float theta) {
    return guarded([&] { rotate(x, size_t(len), size_t(position), size_t(dim), theta); });
}

}  // extern "C"
