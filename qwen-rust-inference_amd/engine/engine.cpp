// Host engine: a C++ restatement of the reference's Rust device engine
// (src/device.rs) over the qr_* bridge ABI. Citations are to the reference.
// It is the bridge's caller in this repository's tests and benchmark; the
// reference's own Rust engine binds the same bridge unchanged.
#include <dlfcn.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "../../include/qwen_bridge.h"
#include "../../include/qwen_engine.h"

namespace {

thread_local std::string g_error;

struct Error {
    std::string what;
};
void require(bool ok, const std::string& what) {
    if (!ok) throw Error{what};
}
// the message is built only on failure (checks over every element of a
// vector run this once per element)
void require(bool ok, const char* what) {
    if (!ok) throw Error{what};
}
// Every value finite (the reference's NaN/Inf check on device reads and
// uploads): one pass that stops at the first non-finite value.
void require_finite(const float* v, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(v[i])) throw Error{"NaN/Inf detected"};
}
template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const Error& e) {
        g_error = e.what;
    } catch (const std::exception& e) {
        g_error = e.what();
    }
    return -1;
}
int int32(size_t n) {
    require(n <= size_t(INT32_MAX), "count exceeds i32");
    return int(n);
}

// Op codes (src/device.rs:39-73).
enum Op {
    RmsNorm = 1, Add = 2, SiluProduct = 3, ConvSilu = 4, DeltaQk = 5, DeltaGates = 6, DeltaRule = 7,
    AttentionQuery = 8, AttentionKv = 9, AttentionRead = 10, EmbedBf16 = 11, AddRmsNorm = 12, RmsNormGate = 13,
    DeltaRuleGated = 14, AttentionQueryKv = 15, Argmax = 16, EmbedBf16Picked = 17
};

constexpr int kAbi = 3;
constexpr size_t kAttentionSplit = 32;  // ATTENTION_SPLIT (src/device.rs:192)
constexpr size_t kKvBlock = 64;         // KV_BLOCK (src/device.rs:201)
constexpr size_t kPrefillFlush = 32;    // PREFILL_FLUSH_INTERVAL (src/device.rs:858)
constexpr size_t kVerifyRows = 8;       // VERIFY_ROWS (src/device.rs:865)
constexpr size_t kDecodeRowsMax = 4;    // rows of one qr_decode_rows launch
size_t kv_rows(size_t capacity) { return (capacity + kKvBlock - 1) / kKvBlock * kKvBlock; }
size_t score_row(size_t capacity, size_t head_dim) {
    size_t splits = (capacity + kAttentionSplit - 1) / kAttentionSplit;
    size_t b = splits * (head_dim + 2);
    return capacity > b ? capacity : b;
}

// ---------------------------------------------------------------- Api (src/device.rs:249-532)
struct Api {
    void* library = nullptr;
    Context* ctx = nullptr;
    int kind = 0;
    int (*create)(Context**) = nullptr;
    int (*alloc)(Context*, float**, size_t) = nullptr;
    void (*free_)(Context*, float*) = nullptr;
    int (*write)(Context*, float*, const float*, size_t) = nullptr;
    int (*read)(Context*, float*, const float*, size_t) = nullptr;
    int (*copy)(Context*, float*, const float*, size_t) = nullptr;
    int (*run)(Context*, int, int, const Params*) = nullptr;
    int (*gemv)(Context*, float*, const float*, const float*, int, int) = nullptr;
    int (*gemv_bf16)(Context*, float*, const float*, const float*, int, int) = nullptr;
    int (*gemm)(Context*, float*, const float*, const float*, int, int, int) = nullptr;
    int (*gemm_bf16)(Context*, float*, const float*, const float*, int, int, int) = nullptr;
    int (*gemm_i8)(Context*, float*, const float*, const float*, int, int, int) = nullptr;
    using Group = int (*)(Context*, int, const QrProjection*, const float*, int, int);
    using Glu = int (*)(Context*, float*, float*, float*, const float*, const float*, const float*, int, int, int);
    using AddNorm = int (*)(Context*, float*, const float*, const float*, int, int, const QrAddNormPost*);
    Group group_bf16 = nullptr, group_i8 = nullptr, group_f32 = nullptr;
    Glu glu_bf16 = nullptr, glu_i8 = nullptr, glu_f32 = nullptr;
    AddNorm add_norm_bf16 = nullptr, add_norm_i8 = nullptr, add_norm_f32 = nullptr;
    int (*delta_mixer)(Context*, const QrDelta*) = nullptr;
    int (*decode_plan)(Context*, const QrDecodeDesc*, QrDecodePlan**) = nullptr;
    int (*decode_step)(Context*, QrDecodePlan*, int, int) = nullptr;
    int (*decode_step_row)(Context*, QrDecodePlan*, int, int, int, int) = nullptr;
    int (*decode_step_capture)(Context*, QrDecodePlan*, int, int, float*, int64_t) = nullptr;
    int (*decode_accept)(Context*, QrDecodePlan*, int) = nullptr;
    int (*decode_rows)(Context*, QrDecodePlan*, const int32_t*, int, int, int, int) = nullptr;
    int (*decode_steps)(Context*, QrDecodePlan*, int, int, int, int32_t*, float*) = nullptr;
    void (*decode_free)(Context*, QrDecodePlan*) = nullptr;
    int (*embed_rows)(Context*, float*, const float*, int, int, int, const int32_t*, int) = nullptr;
    int (*gemm_f32_prepare)(Context*, const float*, int, int) = nullptr;
    int (*gemm_bf16_prepare)(Context*, const float*, int, int) = nullptr;
    int (*gemm_i8_prepare)(Context*, const float*, int, int) = nullptr;
    int (*profile)(Context*, int) = nullptr;
    long (*profile_read)(Context*, char*, size_t) = nullptr;
    int (*sync_)(Context*) = nullptr;
    const char* (*error)(Context*) = nullptr;
    const char* (*info)(Context*) = nullptr;
    void (*destroy)(Context*) = nullptr;
    int max_op = EmbedBf16;
    bool snapshots = false;
    int argmax = 0;

    ~Api() {
        if (ctx && destroy) destroy(ctx);
        if (library) dlclose(library);
    }
    template <class T>
    T symbol(const char* name, bool mandatory) {
        void* p = dlsym(library, name);
        if (!p && mandatory) {
            const char* e = dlerror();
            throw Error{std::string("missing bridge symbol ") + name + (e ? std::string(": ") + e : "")};
        }
        return reinterpret_cast<T>(p);
    }
    void open(const char* path, int expect_kind, int disable) {
        library = dlopen(path, RTLD_NOW);
        if (!library) {
            const char* e = dlerror();
            throw Error{e ? e : "dynamic loader failed"};
        }
        auto abi = symbol<int (*)()>("qr_abi", true);
        auto bridge_kind = symbol<int (*)()>("qr_kind", true);
        require(abi() == kAbi && bridge_kind() == expect_kind,
                 "bridge ABI/kind mismatch (wrong engine or CPU test bridge)");
        kind = expect_kind;
        create = symbol<decltype(create)>("qr_create", true);
        alloc = symbol<decltype(alloc)>("qr_alloc", true);
        free_ = symbol<decltype(free_)>("qr_free", true);
        write = symbol<decltype(write)>("qr_write", true);
        read = symbol<decltype(read)>("qr_read", true);
        copy = symbol<decltype(copy)>("qr_copy", true);
        run = symbol<decltype(run)>("qr_run", true);
        gemv = symbol<decltype(gemv)>("qr_gemv", true);
        gemv_bf16 = symbol<decltype(gemv_bf16)>("qr_gemv_bf16", true);
        gemm = symbol<decltype(gemm)>("qr_gemm", true);
        gemm_bf16 = symbol<decltype(gemm_bf16)>("qr_gemm_bf16", true);
        sync_ = symbol<decltype(sync_)>("qr_sync", true);
        error = symbol<decltype(error)>("qr_error", true);
        info = symbol<decltype(info)>("qr_info", true);
        destroy = symbol<decltype(destroy)>("qr_destroy", true);
        gemm_i8 = symbol<decltype(gemm_i8)>("qr_gemm_i8", false);
        if (!(disable & QE_NO_FUSIONS)) {
            group_bf16 = symbol<Group>("qr_gemm_bf16_group", false);
            group_i8 = symbol<Group>("qr_gemm_i8_group", false);
            glu_bf16 = symbol<Glu>("qr_gemm_bf16_glu", false);
            glu_i8 = symbol<Glu>("qr_gemm_i8_glu", false);
            add_norm_bf16 = symbol<AddNorm>("qr_gemm_bf16_add_norm", false);
            add_norm_i8 = symbol<AddNorm>("qr_gemm_i8_add_norm", false);
        }
        if (!(disable & QE_NO_F32_FUSIONS)) {
            group_f32 = symbol<Group>("qr_gemm_f32_group", false);
            glu_f32 = symbol<Glu>("qr_gemm_f32_glu", false);
            add_norm_f32 = symbol<AddNorm>("qr_gemm_f32_add_norm", false);
        }
        if (!(disable & QE_NO_DELTA_MIXER)) delta_mixer = symbol<decltype(delta_mixer)>("qr_delta_mixer", false);
        if (!(disable & QE_NO_DECODE_STEP)) {
            decode_plan = symbol<decltype(decode_plan)>("qr_decode_plan", false);
            decode_step = symbol<decltype(decode_step)>("qr_decode_step", false);
            decode_free = symbol<decltype(decode_free)>("qr_decode_plan_free", false);
            decode_steps = symbol<decltype(decode_steps)>("qr_decode_steps", false);
            decode_step_row = symbol<decltype(decode_step_row)>("qr_decode_step_row", false);
            if (!(disable & QE_NO_DECODE_CAPTURE))
                decode_step_capture = symbol<decltype(decode_step_capture)>("qr_decode_step_capture", false);
            if (!(disable & QE_NO_DECODE_ROWS)) decode_rows = symbol<decltype(decode_rows)>("qr_decode_rows", false);
            decode_accept = symbol<decltype(decode_accept)>("qr_decode_accept", false);
            if (!decode_plan || !decode_step || !decode_free) decode_plan = nullptr;
        }
        if (!(disable & QE_NO_EMBED_ROWS)) embed_rows = symbol<decltype(embed_rows)>("qr_embed_rows", false);
        if (!(disable & QE_NO_PREPARED_GEMM)) {
            gemm_f32_prepare = symbol<decltype(gemm_f32_prepare)>("qr_gemm_f32_prepare", false);
            gemm_bf16_prepare = symbol<decltype(gemm_bf16_prepare)>("qr_gemm_bf16_prepare", false);
            gemm_i8_prepare = symbol<decltype(gemm_i8_prepare)>("qr_gemm_i8_prepare", false);
        }
        profile = symbol<decltype(profile)>("qr_profile", false);
        profile_read = symbol<decltype(profile_read)>("qr_profile_read", false);
        if (!(disable & QE_NO_SNAPSHOTS)) {
            auto f = symbol<int (*)()>("qr_snapshots", false);
            snapshots = f && f() == 1;
        }
        if (!(disable & QE_NO_ARGMAX)) {
            auto f = symbol<int (*)()>("qr_argmax", false);
            argmax = f ? f() : 0;
        }
        if (!(disable & QE_NO_FUSED_OPS)) {
            auto f = symbol<int (*)()>("qr_max_op", false);
            max_op = f ? f() : EmbedBf16;
        }
        Context* c = nullptr;
        int status = create(&c);
        require(status == 0 && c, "bridge context creation failed, status=" + std::to_string(status));
        ctx = c;
        if ((disable & QE_DECODE_RESIDENCY_TEST) && decode_plan) {
            auto set_option = symbol<int (*)(Context*, const char*, int)>("qr_set_option", false);
            if (!set_option || set_option(ctx, "decode_residency_test", 1) != 0) decode_plan = nullptr;
        }
        if ((disable & QE_NO_PLAIN_DECODE_LAUNCH) && decode_plan) {
            auto set_option = symbol<int (*)(Context*, const char*, int)>("qr_set_option", false);
            if (!set_option || set_option(ctx, "decode_cooperative", 1) != 0) decode_plan = nullptr;
        }
    }
    void check(int status) const {
        if (status == 0) return;
        throw Error{std::string("bridge: ") + error(ctx) + " (status=" + std::to_string(status) + ")"};
    }
    bool runs(int op) const { return op <= max_op; }
    void sync() const { check(sync_(ctx)); }
    void op(int code, size_t count, std::initializer_list<float*> p, std::initializer_list<size_t> n,
            std::initializer_list<float> f) const {
        Params a{};
        int i = 0;
        for (float* v : p) a.p[i++] = v;
        i = 0;
        for (size_t v : n) a.n[i++] = int32(v);
        i = 0;
        for (float v : f) a.f[i++] = v;
        check(run(ctx, code, int32(count), &a));
    }
};

// A device allocation owned by the engine (src/device.rs:586-647).
struct Buffer {
    const Api* api = nullptr;
    float* p = nullptr;
    size_t len = 0;
    Buffer() = default;
    Buffer(const Api* a, size_t n) : api(a), len(n) {
        require(n > 0 && n <= size_t(INT32_MAX), "device allocation overflow/empty");
        api->check(api->alloc(api->ctx, &p, n));
        require(p != nullptr, "null device allocation");
    }
    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;
    Buffer(Buffer&& o) noexcept { *this = std::move(o); }
    Buffer& operator=(Buffer&& o) noexcept {
        if (this != &o) {
            release();
            api = o.api;
            p = o.p;
            len = o.len;
            o.p = nullptr;
            o.len = 0;
        }
        return *this;
    }
    ~Buffer() { release(); }
    void release() {
        if (p && api) api->free_(api->ctx, p);
        p = nullptr;
    }
    float* at(size_t offset) const {
        require(offset < len, "device buffer offset");
        return p + offset;
    }
    void write(const float* v, size_t n) const {
        require(n > 0 && n <= len, "device write bounds");
        api->check(api->write(api->ctx, p, v, n));
    }
    std::vector<float> read(size_t n) const {
        require(n > 0 && n <= len, "device read bounds");
        std::vector<float> host(n);
        api->check(api->read(api->ctx, host.data(), p, n));
        require_finite(host.data(), host.size());
        return host;
    }
};

Buffer upload(const Api* api, const float* v, size_t n) {
    require_finite(v, n);
    Buffer b(api, n);
    b.write(v, n);
    return b;
}
Buffer upload_words(const Api* api, const std::vector<uint32_t>& words) {
    Buffer b(api, words.size());
    api->check(api->write(api->ctx, b.p, reinterpret_cast<const float*>(words.data()), words.size()));
    return b;
}

// quantize_int8_rows (src/device.rs:220-239).
void quantize_rows(const float* w, size_t rows, size_t cols, float* scales, int8_t* q) {
    for (size_t r = 0; r < rows; ++r) {
        const float* row = w + r * cols;
        float max = 0.f;
        for (size_t j = 0; j < cols; ++j) max = std::fmax(max, std::fabs(row[j]));
        const float scale = max / 127.f;
        scales[r] = scale;
        for (size_t j = 0; j < cols; ++j) {
            if (scale == 0.f) {
                q[r * cols + j] = 0;
                continue;
            }
            float v = std::nearbyint(row[j] / scale);  // round half to even
            q[r * cols + j] = int8_t(std::fmin(127.f, std::fmax(-127.f, v)));
        }
    }
}

bool bf16_exact(float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    return (b & 0xffff) == 0;
}

// DeviceMatrix (src/device.rs:648-768).
struct DeviceMatrix {
    Buffer buffer;
    size_t rows = 0, cols = 0;
    bool bf16 = false, int8 = false;
    bool f32() const { return !bf16 && !int8; }
    size_t bytes() const { return int8 ? rows * cols + 4 * rows : rows * cols * (bf16 ? 2 : 4); }

    static DeviceMatrix make(const Api* api, const float* w, size_t rows, size_t cols, int format) {
        int32(rows);
        int32(cols);
        DeviceMatrix m;
        m.rows = rows;
        m.cols = cols;
        const size_t n = rows * cols;
        if (format == QE_INT8) {
            require(api->gemm_i8 != nullptr, "int8 weights need a bridge with qr_gemm_i8");
            std::vector<float> scales(rows);
            std::vector<int8_t> q(n);
            quantize_rows(w, rows, cols, scales.data(), q.data());
            // upload_int8 (src/device.rs:550-561): scales, then 4 values per word.
            std::vector<uint32_t> words(rows + (n + 3) / 4, 0u);
            for (size_t r = 0; r < rows; ++r) std::memcpy(&words[r], &scales[r], 4);
            for (size_t i = 0; i < n; ++i) words[rows + i / 4] |= uint32_t(uint8_t(q[i])) << (8 * (i % 4));
            m.buffer = upload_words(api, words);
            m.int8 = true;
            return m;
        }
        bool exact = format == QE_BF16_EXACT;
        for (size_t i = 0; exact && i < n; ++i) exact = bf16_exact(w[i]);
        if (exact) {
            // upload_bf16_bits (src/device.rs:535-549): element 2i in the low half.
            std::vector<uint32_t> words((n + 1) / 2, 0u);
            for (size_t i = 0; i < n; ++i) {
                uint32_t b;
                std::memcpy(&b, &w[i], 4);
                words[i / 2] |= (b >> 16) << (16 * (i % 2));
            }
            m.buffer = upload_words(api, words);
            m.bf16 = true;
            return m;
        }
        m.buffer = upload(api, w, n);
        return m;
    }
    // project (src/device.rs:724-768): Y[t, rows] = X[t, cols] . W^T
    void project(const Buffer& x, const Buffer& out, size_t tokens) const {
        require(tokens > 0 && x.len >= tokens * cols && out.len >= tokens * rows, "device GEMV shape");
        const Api* a = buffer.api;
        int r = int32(rows), c = int32(cols), t = int32(tokens);
        if (int8) {
            require(a->gemm_i8 != nullptr, "bridge has no qr_gemm_i8");
            a->check(a->gemm_i8(a->ctx, out.p, buffer.p, x.p, r, c, t));
        } else if (tokens == 1) {
            a->check((bf16 ? a->gemv_bf16 : a->gemv)(a->ctx, out.p, buffer.p, x.p, r, c));
        } else {
            a->check((bf16 ? a->gemm_bf16 : a->gemm)(a->ctx, out.p, buffer.p, x.p, r, c, t));
        }
    }
};

// project_all (src/device.rs:769-816), with the fp32 arm.
void project_all(const Api* a, const Buffer& x, const std::vector<std::pair<const DeviceMatrix*, const Buffer*>>& items,
                 size_t tokens) {
    if (items.empty()) return;
    const DeviceMatrix* first = items[0].first;
    bool same_cols = items.size() > 1;
    bool all_bf16 = true, all_i8 = true, all_f32 = true;
    for (auto& it : items) {
        same_cols = same_cols && it.first->cols == first->cols;
        all_bf16 = all_bf16 && it.first->bf16;
        all_i8 = all_i8 && it.first->int8;
        all_f32 = all_f32 && it.first->f32();
    }
    Api::Group group = all_bf16 ? a->group_bf16 : all_i8 ? a->group_i8 : all_f32 ? a->group_f32 : nullptr;
    if (!group || !same_cols) {
        for (auto& it : items) it.first->project(x, *it.second, tokens);
        return;
    }
    std::vector<QrProjection> entries;
    for (auto& it : items) {
        require(tokens > 0 && x.len >= tokens * it.first->cols && it.second->len >= tokens * it.first->rows,
                "device GEMV shape");
        entries.push_back(QrProjection{it.second->p, it.first->buffer.p, int32(it.first->rows)});
    }
    a->check(group(a->ctx, int32(entries.size()), entries.data(), x.p, int32(first->cols), int32(tokens)));
}

struct AttentionCfg {
    size_t heads, kv_heads, head_dim, rotary_dim;
    float theta, eps;
};
struct DeltaCfg {
    size_t key_heads, value_heads, key_dim, value_dim, kernel;
    float eps;
};

// DeviceBlock / DeviceMixer (src/device.rs:817-854).
struct DeviceBlock {
    Buffer input, post;
    DeviceMatrix gate, up, down;
    float eps = 0.f;
    bool attention = false;
    // attention
    AttentionCfg ac{};
    DeviceMatrix q, k, v, o;
    Buffer qn, kn, qkn;
    // delta
    DeltaCfg dc{};
    DeviceMatrix qkv, z, a, b, out;
    Buffer conv, dt, alog, gates, norm;
};

}  // namespace

// DeviceModel (src/device.rs:866-1297).
struct QeModel {
    std::unique_ptr<Api> api;
    QwConfig config{};
    DeviceMatrix embedding;
    std::optional<DeviceMatrix> lm_head;
    Buffer norm;
    std::vector<DeviceBlock> blocks;
    uint64_t run_budget = uint64_t(4) << 30;  // MAX_RUN_BYTES
    std::string info;
    // Runs hold the model (the reference's DeviceRun borrows it, so it
    // outlives them): qe_model_free marks it, the last run's free releases it.
    std::atomic<int> runs{0};
    bool released = false;

    const DeviceMatrix& output() const { return lm_head ? *lm_head : embedding; }

    size_t delta_state_bytes() const {
        size_t total = 0;
        for (auto& b : blocks)
            if (!b.attention)
                total += 4 * (std::max<size_t>(b.qkv.rows * (b.dc.kernel - 1), 1) +
                              b.dc.value_heads * b.dc.key_dim * b.dc.value_dim);
        return total;
    }
    // run_bytes_chunked (src/device.rs:1144-1177)
    uint64_t run_bytes(size_t capacity, size_t chunk) const {
        uint64_t floats = 0;
        for (auto& b : blocks) {
            if (b.attention) {
                size_t q = b.ac.heads * b.ac.head_dim, kv = b.ac.kv_heads * b.ac.head_dim;
                floats += uint64_t(kv_rows(capacity)) * 2 * kv + uint64_t(score_row(capacity, b.ac.head_dim)) * b.ac.heads +
                          uint64_t(chunk) * (q * 4 + kv * 2) + uint64_t((chunk + 7) / 8 * 8) * q;
            } else {
                size_t q = b.dc.value_heads * b.dc.key_dim, v = b.dc.value_heads * b.dc.value_dim;
                floats += uint64_t(b.qkv.rows * std::max<size_t>(b.dc.kernel - 1, 1) +
                                   b.dc.value_heads * b.dc.key_dim * b.dc.value_dim) +
                          uint64_t(chunk) * (b.qkv.rows * 2 + q * 2 + b.dc.value_heads * 4 + v * 4);
            }
        }
        size_t h = size_t(config.hidden_size), i = size_t(config.intermediate_size);
        floats += uint64_t(chunk) * (h * 5 + i * 3) + uint64_t(config.vocab_size) * std::min(kVerifyRows, chunk);
        return floats * 4;
    }
};

namespace {

// MixerRun (src/device.rs:1296-1329).
struct MixerRun {
    bool attention = false;
    Buffer mixed, key, value, query, gate, context, keys, values, scores;
    Buffer projected, convolved, conv_state, recurrent, dquery, dkey, a, b, z, decay, beta, core, normalized, gated;
};

struct Record {
    qe_record_fn fn;
    void* user;
};

}  // namespace

struct QeCheckpoint {
    size_t position = 0;
    std::vector<std::optional<std::pair<std::vector<float>, std::vector<float>>>> delta;  // (conv, recurrent)
};

// DeviceRun (src/device.rs:1330-2566).
struct QeRun {
    QeModel* model = nullptr;
    size_t capacity = 0, chunk = 0, snapshots = 0, snapshot_rows = 0;
    std::optional<std::pair<size_t, size_t>> pending;
    size_t position = 0;
    bool failed = false;
    std::vector<MixerRun> mixers;
    Buffer x, norm, mixed, residual, gate, up, product, ffn, logits, picks;
    Buffer captured;  // the one-launch step's per-layer records (qr_decode_step_capture), made on first use
    bool greedy_rows = false;
    std::vector<uint32_t> picked;
    size_t pick_slot = 0;
    bool logits_unread = false;
    // The bridge's one-launch decode step over this run's buffers (fp32
    // matrices only), used by forward for uncaptured one-token steps.
    QrDecodePlan* plan = nullptr;
    // The weight-edit overlay (set_edit, src/device.rs:1401-1438): the
    // validated edits and host fp32 copies of the down matrices of the edited
    // layers ([hidden, intermediate] row-major); applied by forward_body.
    struct EditEntry {
        size_t layer;
        std::vector<size_t> columns;
        std::vector<float> direction;  // empty: disable the units
        float coefficient;
    };
    std::vector<EditEntry> edits;
    std::vector<std::vector<float>> edit_down;  // per layer; empty when not edited
    bool edited(size_t layer) const { return layer < edit_down.size() && !edit_down[layer].empty(); }

    const Api* api() const { return model->api.get(); }
    ~QeRun() { drop_plan(); }
    void drop_plan() {
        if (plan && model) api()->decode_free(api()->ctx, plan);
        plan = nullptr;
    }
    // qr_decode_plan over the run's buffers; a bridge that declines the shape
    // leaves the run on the op sequence.
    void make_plan() {
        drop_plan();
        const Api* a = api();
        const QwConfig& c = model->config;
        if (!a->decode_plan || model->embedding.int8) return;
        // all matrices fp32, all BF16 (a BF16-exact model: the tied LM head is
        // the BF16 embedding table), or all int8 (the int8 model's LM head is
        // int8 too)
        const bool q8 = model->output().int8, b16 = model->output().bf16;
        auto ok = [q8, b16](const DeviceMatrix& m) { return q8 ? m.int8 : b16 ? m.bf16 : m.f32(); };
        if (!ok(model->output())) return;
        std::vector<QrDecodeLayer> layers;
        const DeviceBlock* attn = nullptr;
        const DeviceBlock* delta = nullptr;
        // The plan carries one eps for every norm (block, q/k, gated) and one
        // attention / DeltaNet geometry: decline it unless every block agrees.
        const float eps = c.rms_norm_eps;
        for (const DeviceBlock& b : model->blocks) {
            if (b.eps != eps) return;
            if (b.attention) {
                if (b.ac.eps != eps) return;
                if (attn && (b.ac.heads != attn->ac.heads || b.ac.kv_heads != attn->ac.kv_heads ||
                             b.ac.head_dim != attn->ac.head_dim || b.ac.rotary_dim != attn->ac.rotary_dim ||
                             b.ac.theta != attn->ac.theta))
                    return;
                attn = &b;
            } else {
                if (b.dc.eps != eps) return;
                if (delta && (b.dc.key_heads != delta->dc.key_heads || b.dc.value_heads != delta->dc.value_heads ||
                              b.dc.key_dim != delta->dc.key_dim || b.dc.value_dim != delta->dc.value_dim ||
                              b.dc.kernel != delta->dc.kernel))
                    return;
                delta = &b;
            }
        }
        for (size_t l = 0; l < model->blocks.size(); ++l) {
            const DeviceBlock& b = model->blocks[l];
            MixerRun& m = mixers[l];
            if (!ok(b.gate) || !ok(b.up) || !ok(b.down)) return;
            QrDecodeLayer d{};
            d.attention = b.attention ? 1 : 0;
            d.input_norm = b.input.p;
            d.post_norm = b.post.p;
            d.gate = b.gate.buffer.p;
            d.up = b.up.buffer.p;
            d.down = b.down.buffer.p;
            if (b.attention) {
                if (!ok(b.q) || !ok(b.k) || !ok(b.v) || !ok(b.o)) return;
                d.q = b.q.buffer.p;
                d.k = b.k.buffer.p;
                d.v = b.v.buffer.p;
                d.o = b.o.buffer.p;
                d.qk_norm = b.qkn.p;
                d.keys = m.keys.p;
                d.values = m.values.p;
            } else {
                if (!ok(b.qkv) || !ok(b.z) || !ok(b.a) || !ok(b.b) || !ok(b.out)) return;
                d.qkv = b.qkv.buffer.p;
                d.z = b.z.buffer.p;
                d.a = b.a.buffer.p;
                d.b = b.b.buffer.p;
                d.conv_w = b.conv.p;
                d.gates = b.gates.p;
                d.norm_w = b.norm.p;
                d.out = b.out.buffer.p;
                d.conv_state = m.conv_state.p;
                d.recurrent = m.recurrent.p;
            }
            layers.push_back(d);
        }
        QrDecodeDesc desc{};
        desc.hidden = c.hidden_size;
        desc.intermediate = c.intermediate_size;
        desc.vocab = c.vocab_size;
        desc.layers = int32(layers.size());
        desc.heads = attn ? int32(attn->ac.heads) : c.num_heads;
        desc.kv_heads = attn ? int32(attn->ac.kv_heads) : c.num_kv_heads;
        desc.head_dim = attn ? int32(attn->ac.head_dim) : c.head_dim;
        desc.rotary_dim = attn ? int32(attn->ac.rotary_dim) : c.rotary_dim;
        desc.key_heads = delta ? int32(delta->dc.key_heads) : c.key_heads;
        desc.value_heads = delta ? int32(delta->dc.value_heads) : c.value_heads;
        desc.key_dim = delta ? int32(delta->dc.key_dim) : c.key_dim;
        desc.value_dim = delta ? int32(delta->dc.value_dim) : c.value_dim;
        desc.conv_kernel = delta ? int32(delta->dc.kernel) : c.conv_kernel;
        desc.capacity = int32(capacity);
        desc.eps = c.rms_norm_eps;
        desc.theta = attn ? attn->ac.theta : c.rope_theta;
        desc.embedding = model->embedding.buffer.p;
        desc.lm_head = model->output().buffer.p;
        desc.final_norm = model->norm.p;
        desc.logits = logits.p;
        desc.picks = picks.p;
        desc.layer = layers.data();
        desc.weights = q8 ? QR_DECODE_INT8 : b16 ? QR_DECODE_BF16 : QR_DECODE_F32;
        desc.embedding_bf16 = model->embedding.bf16 ? 1 : 0;
        desc.rows = int32(std::min(kVerifyRows, chunk));
        desc.snapshots = int32(snapshots);
        QrDecodePlan* p = nullptr;
        if (a->decode_plan(a->ctx, &desc, &p) == 0) plan = p;
    }
    // EditManifest::apply (src/edit.rs:59-110) on one row of the FFN product:
    // units of the direction-less edits scaled by (1 - coefficient), then the
    // correction -coefficient * d (d . w_j) / (d . d) * product[j] summed over
    // the direction edits' columns j (w_j: column j of down).
    std::vector<float> apply_edit(size_t layer, float* product) const {
        const size_t h = size_t(model->config.hidden_size), i_size = size_t(model->config.intermediate_size);
        const std::vector<float>& down = edit_down[layer];
        for (const EditEntry& e : edits)
            if (e.layer == layer && e.direction.empty())
                for (size_t j : e.columns) product[j] *= 1.f - e.coefficient;
        std::vector<float> correction(h, 0.f);
        for (const EditEntry& e : edits) {
            if (e.layer != layer || e.direction.empty()) continue;
            const std::vector<float>& d = e.direction;
            float denominator = -0.f;
            for (float v : d) denominator += v * v;
            for (size_t j : e.columns) {
                float dot = -0.f;
                for (size_t r = 0; r < h; ++r) dot += d[r] * down[r * i_size + j];
                const float projection = dot / denominator;
                for (size_t r = 0; r < h; ++r) correction[r] -= e.coefficient * d[r] * projection * product[j];
            }
        }
        require_finite(correction.data(), correction.size());
        return correction;
    }

    // One uncaptured token through the plan (the work of forward_body for
    // t == 1, logit_rows == 1): logits and [argmax, non-finite count] land in
    // the run's logits / picks buffers.
    std::vector<float> forward_planned(uint32_t id) {
        const Api* a = api();
        a->check(a->decode_step(a->ctx, plan, int(id), int(position)));
        std::vector<float> out;
        std::vector<float> pk(2);
        a->check(a->read(a->ctx, pk.data(), picks.p, 2));
        require(pk[1] < 1e30f, "one-launch decode step timed out at a stage barrier");
        if (greedy_rows) {
            picked = picks_of(pk, 0, 1);  // the pick is in the read just made
        } else {
            out = logits.read(size_t(model->config.vocab_size));
        }
        position += 1;
        return out;
    }
    // One captured token through the plan (qr_decode_step_capture): the
    // records forward_body would report, in its order (src/device.rs:1748-1761),
    // from one read of the step's record buffer.
    std::vector<float> forward_planned_capture(uint32_t id, const Record* rec) {
        const Api* a = api();
        const size_t h = size_t(model->config.hidden_size), i_size = size_t(model->config.intermediate_size);
        const size_t layers = model->blocks.size(), per = 6 * h + i_size, n = layers * per + h;
        if (captured.len < n) captured = Buffer(a, n);
        a->check(a->decode_step_capture(a->ctx, plan, int(id), int(position), captured.p, int64_t(captured.len)));
        std::vector<float> pk(2);
        a->check(a->read(a->ctx, pk.data(), picks.p, 2));
        require(pk[1] < 1e30f, "one-launch decode step timed out at a stage barrier");
        const std::vector<float> v = captured.read(n);
        static const char* names[] = {"input_norm", "mixed", "after_mixer", "post_norm", "ffn_product", "ffn", "output"};
        const size_t off[] = {0, h, 2 * h, 3 * h, 4 * h, 4 * h + i_size, 5 * h + i_size};
        const size_t len[] = {h, h, h, h, i_size, h, h};
        for (size_t l = 0; l < layers; ++l)
            for (int k = 0; k < 7; ++k) rec->fn(rec->user, int(l), names[k], v.data() + l * per + off[k], int64_t(len[k]));
        std::vector<float> out;
        if (greedy_rows) {
            picked = picks_of(pk, 0, 1);
        } else {
            out = logits.read(size_t(model->config.vocab_size));
        }
        rec->fn(rec->user, int(layers) - 1, "normalized", v.data() + layers * per, int64_t(h));
        if (!out.empty()) rec->fn(rec->user, int(layers) - 1, "logits", out.data(), int64_t(out.size()));
        position += 1;
        return out;
    }
    // The rows of a verify pass through the plan, one launch per row (the
    // decode step of each row's position, so every row equals the sequential
    // decode step bit for bit, as the reference requires of verify rows,
    // src/device.rs:1514-1531): row r's logits / picks in row r of the run's
    // buffers, the DeltaNet states after row r in snapshot copy r + 1 for
    // r < snapshot_rows (what accept restores). The launches are queued back
    // to back; the host reads once at the end.
    // Verify rows: up to four per launch with the weights read once
    // (qr_decode_rows), else one launch per row; either way each row is the
    // decode step of its position bit for bit.
    std::vector<float> forward_planned_rows(const uint32_t* ids, size_t t) {
        const Api* a = api();
        for (size_t r = 0; r < t;) {
            const size_t n = std::min<size_t>(kDecodeRowsMax, t - r);
            if (a->decode_rows && n > 1) {
                int32_t tok[kDecodeRowsMax];
                for (size_t k = 0; k < n; ++k) tok[k] = int32_t(ids[r + k]);
                a->check(a->decode_rows(a->ctx, plan, tok, int(n), int(position + r), int(r), int(snapshot_rows)));
                r += n;
            } else {
                a->check(a->decode_step_row(a->ctx, plan, int(ids[r]), int(position + r), int(r),
                                            r < snapshot_rows ? int(r + 1) : 0));
                ++r;
            }
        }
        std::vector<float> out;
        std::vector<float> pk(2 * t);
        a->check(a->read(a->ctx, pk.data(), picks.p, pk.size()));
        for (size_t r = 0; r < t; ++r) require(pk[2 * r + 1] < 1e30f, "one-launch decode step timed out at a stage barrier");
        if (greedy_rows) {
            picked = picks_of(pk, 0, t);
        } else {
            out = logits.read(size_t(model->config.vocab_size) * t);
        }
        position += t;
        return out;
    }

    // new_run_with (src/device.rs:1198-1294)
    void build(size_t cap, size_t ch, size_t snaps) {
        const QwConfig& c = model->config;
        require(cap > 0 && cap <= size_t(c.max_positions), "device capacity must be 1..=model context limit");
        require(ch > 0, "device prefill chunk must be positive");
        ch = std::min(ch, cap);
        uint64_t bytes = model->run_bytes(cap, ch) + uint64_t(snaps) * model->delta_state_bytes();
        require(bytes <= model->run_budget, "device run for capacity " + std::to_string(cap) + " needs " +
                                                std::to_string(bytes) + " bytes > budget " +
                                                std::to_string(model->run_budget));
        const Api* a = api();
        capacity = cap;
        chunk = ch;
        snapshots = snaps;
        mixers.clear();
        for (auto& b : model->blocks) {
            MixerRun m;
            m.attention = b.attention;
            if (b.attention) {
                size_t q = b.ac.heads * b.ac.head_dim, kv = b.ac.kv_heads * b.ac.head_dim;
                m.mixed = Buffer(a, ch * q * 2);
                m.key = Buffer(a, ch * kv);
                m.value = Buffer(a, ch * kv);
                m.query = Buffer(a, (ch + 7) / 8 * 8 * q);
                m.gate = Buffer(a, ch * q);
                m.context = Buffer(a, ch * q);
                m.keys = Buffer(a, kv_rows(cap) * kv);
                m.values = Buffer(a, kv_rows(cap) * kv);
                m.scores = Buffer(a, score_row(cap, b.ac.head_dim) * b.ac.heads);
            } else {
                size_t q = b.dc.value_heads * b.dc.key_dim, v = b.dc.value_heads * b.dc.value_dim;
                m.projected = Buffer(a, ch * b.qkv.rows);
                m.convolved = Buffer(a, ch * b.qkv.rows);
                m.conv_state = Buffer(a, std::max<size_t>(b.qkv.rows * (b.dc.kernel - 1), 1) * (1 + snaps));
                m.recurrent = Buffer(a, b.dc.value_heads * b.dc.key_dim * b.dc.value_dim * (1 + snaps));
                m.dquery = Buffer(a, ch * q);
                m.dkey = Buffer(a, ch * q);
                m.a = Buffer(a, ch * b.dc.value_heads);
                m.b = Buffer(a, ch * b.dc.value_heads);
                m.z = Buffer(a, ch * v);
                m.decay = Buffer(a, ch * b.dc.value_heads);
                m.beta = Buffer(a, ch * b.dc.value_heads);
                m.core = Buffer(a, ch * v);
                m.normalized = Buffer(a, ch * v);
                m.gated = Buffer(a, ch * v);
            }
            mixers.push_back(std::move(m));
        }
        size_t h = size_t(c.hidden_size), i = size_t(c.intermediate_size);
        x = Buffer(a, ch * h);
        norm = Buffer(a, ch * h);
        mixed = Buffer(a, ch * h);
        residual = Buffer(a, ch * h);
        gate = Buffer(a, ch * i);
        up = Buffer(a, ch * i);
        product = Buffer(a, ch * i);
        ffn = Buffer(a, ch * h);
        logits = Buffer(a, size_t(c.vocab_size) * std::min(kVerifyRows, ch));
        picks = Buffer(a, 2 * kVerifyRows);
        position = 0;
        failed = false;
        pending.reset();
        snapshot_rows = 0;
        greedy_rows = false;
        picked.clear();
        pick_slot = 0;
        logits_unread = false;
        make_plan();
    }

    // step (src/device.rs:1440-1451)
    std::vector<float> step(uint32_t id, const Record* rec) {
        require(!failed, "device run failed; reset required");
        require(id < uint32_t(model->config.vocab_size) && position < capacity, "device token/capacity out of bounds");
        try {
            return forward(&id, 1, rec, 1);
        } catch (...) {
            failed = true;
            throw;
        }
    }

    // prefill (src/device.rs:1456-1490)
    std::optional<std::vector<float>> prefill(const uint32_t* ids, size_t n) {
        bool ok = !failed && n <= capacity - position;
        for (size_t i = 0; ok && i < n; ++i) ok = ids[i] < uint32_t(model->config.vocab_size);
        require(ok, "device prefill token/capacity/failed");
        std::optional<std::vector<float>> last;
        size_t unsynced = 0, chunks = (n + chunk - 1) / chunk;
        for (size_t i = 0; i < chunks; ++i) {
            const bool final_chunk = i + 1 == chunks;
            const size_t len = std::min(chunk, n - i * chunk);
            unsynced += len;
            try {
                auto logits_out = forward(ids + i * chunk, len, nullptr, final_chunk ? 1 : 0);
                if (!final_chunk && unsynced >= kPrefillFlush) {
                    unsynced = 0;
                    api()->sync();
                }
                if (final_chunk) last = std::move(logits_out);
            } catch (...) {
                failed = true;
                throw;
            }
        }
        return last;
    }

    // verify (src/device.rs:1495-1513)
    std::vector<float> verify(const uint32_t* ids, size_t n) {
        bool ok = !failed && n > 0 && n <= std::min(kVerifyRows, chunk) && n <= capacity - position;
        for (size_t i = 0; ok && i < n; ++i) ok = ids[i] < uint32_t(model->config.vocab_size);
        require(ok, "device verify rows/capacity/failed");
        try {
            return forward(ids, n, nullptr, n);
        } catch (...) {
            failed = true;
            throw;
        }
    }
    // verify_rollback (src/device.rs:1514-1531)
    std::vector<float> verify_rollback(const uint32_t* ids, size_t n) {
        require(n > 0 && n <= snapshots + 1, "verify_rollback: more rows than snapshots + 1");
        size_t start = position;
        snapshot_rows = n - 1;
        std::vector<float> out;
        try {
            out = verify(ids, n);
        } catch (...) {
            snapshot_rows = 0;
            throw;
        }
        snapshot_rows = 0;
        pending = std::make_pair(start, n);
        return out;
    }
    // pick_rows / read_picks (src/device.rs:1533-1564)
    void pick_rows(size_t rows) {
        size_t v = size_t(model->config.vocab_size);
        require(pick_slot + rows <= kVerifyRows, "argmax rows beyond the picks buffer");
        api()->op(Argmax, rows, {picks.at(2 * pick_slot), logits.p}, {v}, {});
        picked = read_picks(pick_slot, rows);
    }
    std::vector<uint32_t> read_picks(size_t slot, size_t rows) const {
        std::vector<float> all(2 * (slot + rows));
        api()->check(api()->read(api()->ctx, all.data(), picks.p, all.size()));
        return picks_of(all, slot, rows);
    }
    // rows slot .. slot + rows - 1 of the picks buffer's (index, flag) pairs
    std::vector<uint32_t> picks_of(const std::vector<float>& all, size_t slot, size_t rows) const {
        size_t v = size_t(model->config.vocab_size);
        std::vector<uint32_t> out;
        for (size_t r = slot; r < slot + rows; ++r) {
            float idx = all[2 * r], bad = all[2 * r + 1];
            require(bad == 0.f && idx >= 0.f && size_t(idx) < v, "non-finite logits");
            out.push_back(uint32_t(idx));
        }
        return out;
    }
    // select (src/generate.rs:30-41)
    static uint32_t select_greedy(const std::vector<float>& logits) {
        require_finite(logits.data(), logits.size());
        size_t best = 0;
        for (size_t i = 1; i < logits.size(); ++i)
            if (logits[i] > logits[best]) best = i;
        return uint32_t(best);
    }
    // step_greedy (src/device.rs:1568-1584)
    uint32_t step_greedy(uint32_t id) {
        if (api()->argmax < 1) {
            auto l = step(id, nullptr);
            logits_unread = true;
            return select_greedy(l);
        }
        greedy_rows = true;
        try {
            step(id, nullptr);
        } catch (...) {
            greedy_rows = false;
            throw;
        }
        greedy_rows = false;
        return picked.at(0);
    }
    std::vector<uint32_t> verify_rollback_greedy(const uint32_t* ids, size_t n) {
        if (api()->argmax < 1) {
            auto l = verify_rollback(ids, n);
            size_t v = size_t(model->config.vocab_size);
            std::vector<uint32_t> out;
            for (size_t r = 0; r < n; ++r)
                out.push_back(select_greedy(std::vector<float>(l.begin() + long(r * v), l.begin() + long((r + 1) * v))));
            return out;
        }
        greedy_rows = true;
        try {
            verify_rollback(ids, n);
        } catch (...) {
            greedy_rows = false;
            throw;
        }
        greedy_rows = false;
        std::vector<uint32_t> out;
        out.swap(picked);
        return out;
    }
    // Whether greedy steps from the current position can run as chained
    // one-launch steps (forward's one-launch conditions, nothing pending);
    // chained_greedy refuses a count past the run's capacity before any launch.
    bool can_chain() const {
        return plan && edits.empty() && api()->decode_steps && snapshot_rows == 0 && pick_slot == 0;
    }
    // `count` greedy steps from token `first` at the current position, queued
    // back to back with one read-back: next[i] is the pick after step i (the
    // token step i + 1 feeds). Seconds of the call.
    double chained_greedy(uint32_t first, size_t count, uint32_t* next) {
        const Api* a = api();
        require(!failed, "device run failed; reset required");
        require(first < uint32_t(model->config.vocab_size) && position + count <= capacity,
                "device token/capacity out of bounds");
        std::vector<int32_t> got(count);
        float bad = 0.f;
        pending.reset();
        auto t0 = std::chrono::steady_clock::now();
        const int st = a->decode_steps(a->ctx, plan, int(first), int(position), int(count), got.data(), &bad);
        const double total = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        position += count;
        logits_unread = true;
        if (st != 0 || bad != 0.f) failed = true;
        a->check(st);
        require(bad < 1e30f, "one-launch decode step timed out at a stage barrier");
        require(bad == 0.f, "non-finite logits");
        for (size_t i = 0; i < count; ++i) next[i] = uint32_t(got[i]);
        picked = {next[count - 1]};
        return total;
    }
    // accept (src/device.rs:1626-1662)
    void accept(size_t rows) {
        require(pending.has_value(), "accept needs a verify_rollback pass");
        auto [start, t] = *pending;
        pending.reset();
        require(rows >= 1 && rows <= t, "accept rows out of range");
        if (rows == t) return;
        const Api* a = api();
        if (plan && a->decode_accept && rows <= snapshots) {  // the same copies in one launch
            a->check(a->decode_accept(a->ctx, plan, int(rows)));
            position = start + rows;
            return;
        }
        for (size_t l = 0; l < model->blocks.size(); ++l) {
            const DeviceBlock& b = model->blocks[l];
            if (b.attention) continue;
            MixerRun& m = mixers[l];
            size_t state = b.dc.value_heads * b.dc.key_dim * b.dc.value_dim;
            size_t conv = std::max<size_t>(b.qkv.rows * (b.dc.kernel - 1), 1);
            a->check(a->copy(a->ctx, m.recurrent.p, m.recurrent.at(rows * state), state));
            if (b.dc.kernel > 1) a->check(a->copy(a->ctx, m.conv_state.p, m.conv_state.at(rows * conv), conv));
        }
        position = start + rows;
    }

    // forward (src/device.rs:1703-1737)
    std::vector<float> forward(const uint32_t* ids, size_t t, const Record* rec, size_t logit_rows) {
        pending.reset();
        require(t > 0 && t <= chunk && (!rec || t == 1) && (logit_rows <= 1 || logit_rows == t),
                "device forward chunk/capture");
        const Api* a = api();
        if (plan && edits.empty() && t == 1 && !rec && logit_rows == 1 && snapshot_rows == 0 && pick_slot == 0) {
            auto out = forward_planned(ids[0]);
            logits_unread = greedy_rows;
            return out;
        }
        if (plan && edits.empty() && a->decode_step_capture && t == 1 && rec && logit_rows == 1 &&
            snapshot_rows == 0 && pick_slot == 0) {
            auto out = forward_planned_capture(ids[0], rec);
            logits_unread = greedy_rows;
            return out;
        }
        if (plan && edits.empty() && a->decode_step_row && t > 1 && !rec && logit_rows == t && pick_slot == 0 &&
            t <= std::min(kVerifyRows, chunk)) {
            auto out = forward_planned_rows(ids, t);
            logits_unread = false;
            return out;
        }
        size_t h = size_t(model->config.hidden_size);
        if (a->embed_rows && t > 1) {  // the whole chunk in one call
            std::vector<int32_t> rows(ids, ids + t);
            a->check(a->embed_rows(a->ctx, x.at(0), model->embedding.buffer.p, int(model->config.vocab_size), int(h),
                                   model->embedding.bf16 ? 1 : 0, rows.data(), int(t)));
        }
        for (size_t r = 0; r < t && !(a->embed_rows && t > 1); ++r) {
            float* xr = x.at(r * h);
            if (model->embedding.bf16) {
                a->op(EmbedBf16, h, {xr, model->embedding.buffer.p}, {size_t(ids[r]), h}, {});
            } else {
                const float* row = model->embedding.buffer.p + size_t(ids[r]) * h;
                a->check(a->copy(a->ctx, xr, row, h));
            }
        }
        auto out = forward_body(t, rec, logit_rows);
        logits_unread = greedy_rows && logit_rows == 1 && t == 1;
        return out;
    }

    // forward_body (src/device.rs:1740-2378)
    std::vector<float> forward_body(size_t t, const Record* rec, size_t logit_rows) {
        const Api* a = api();
        const QwConfig& cfg = model->config;
        const size_t h = size_t(cfg.hidden_size), i_size = size_t(cfg.intermediate_size);
        const bool capture = rec != nullptr;
        auto record = [&](size_t layer, const char* name, const Buffer& b, size_t n) {
            if (!capture) return;
            auto v = b.read(n);
            rec->fn(rec->user, int(layer), name, v.data(), int64_t(n));
        };
        auto norm_op = [&](float* xp, const Buffer& w, float* outp, size_t d, size_t groups, float eps, float offset) {
            a->op(RmsNorm, groups, {outp, xp, w.p}, {d}, {eps, offset});
        };
        const bool fused_add_norm = a->runs(AddRmsNorm);
        auto add_norm = [&](float* sum, float* u, float* v, const Buffer& w, float* outp, float eps) {
            if (fused_add_norm) {
                a->op(AddRmsNorm, t, {sum, u, v, outp, w.p}, {h}, {eps, 1.f});
            } else {
                a->op(Add, h * t, {sum, u, v}, {}, {});
                norm_op(sum, w, outp, h, t, eps, 1.f);
            }
        };
        const bool tail = t == 1 && !capture && fused_add_norm;
        // project_norm (src/device.rs:1792-1836), with the fp32 arm.
        auto project_norm = [&](const DeviceMatrix& m, const Buffer& xin, const Buffer& y, const Buffer& sum,
                                const Buffer& u, const Buffer& v, const Buffer& w, float eps) -> bool {
            Api::AddNorm fused = m.bf16 ? a->add_norm_bf16 : m.int8 ? a->add_norm_i8 : a->add_norm_f32;
            if (!(fused && tail && m.rows == h && xin.len >= m.cols && y.len >= h && sum.len >= h)) {
                m.project(xin, y, t);
                return false;
            }
            QrAddNormPost post{sum.p, u.p, v.p, w.p, norm.p, eps, 1.f};
            a->check(fused(a->ctx, y.p, m.buffer.p, xin.p, int32(m.rows), int32(m.cols), &post));
            return true;
        };
        bool final_normed = false, normed = false;
        for (size_t layer = 0; layer < model->blocks.size(); ++layer) {
            const DeviceBlock& b = model->blocks[layer];
            MixerRun& s = mixers[layer];
            if (!normed) norm_op(x.p, b.input, norm.p, h, t, b.eps, 1.f);
            record(layer, "input_norm", norm, h);
            bool post_normed;
            if (b.attention) {
                const AttentionCfg& c = b.ac;
                project_all(a, norm, {{&b.q, &s.mixed}, {&b.k, &s.key}, {&b.v, &s.value}}, t);
                if (a->runs(AttentionQueryKv)) {
                    a->op(AttentionQueryKv, (c.heads + c.kv_heads) * t,
                          {s.query.p, s.mixed.p, b.qkn.p, s.gate.p, s.keys.p, s.key.p, s.value.p, s.values.p},
                          {c.head_dim, c.rotary_dim, position, c.heads, c.kv_heads, t}, {c.eps, c.theta});
                } else {
                    a->op(AttentionQuery, c.heads * t, {s.query.p, s.mixed.p, b.qn.p, s.gate.p},
                          {c.head_dim, c.rotary_dim, position, c.heads}, {c.eps, c.theta});
                    a->op(AttentionKv, c.kv_heads * t, {s.keys.p, s.key.p, b.kn.p, s.value.p, s.values.p},
                          {c.head_dim, c.rotary_dim, position, c.kv_heads}, {c.eps, c.theta});
                }
                a->op(AttentionRead, c.heads, {s.context.p, s.query.p, s.keys.p, s.values.p, s.gate.p, s.scores.p},
                      {c.head_dim, c.heads, c.kv_heads, position + 1, capacity, t, score_row(capacity, c.head_dim)}, {});
                post_normed = project_norm(b.o, s.context, mixed, residual, x, mixed, b.post, b.eps);
            } else {
                const DeltaCfg& c = b.dc;
                project_all(a, norm, {{&b.qkv, &s.projected}, {&b.z, &s.z}, {&b.a, &s.a}, {&b.b, &s.b}}, t);
                const size_t channels = b.qkv.rows, vd = c.value_heads * c.value_dim, vh = c.value_heads;
                const bool fused = a->delta_mixer && a->runs(DeltaRuleGated) && a->runs(RmsNormGate);
                if (fused && snapshot_rows == 0) {
                    QrDelta d{s.convolved.p, s.projected.p, b.conv.p, s.conv_state.p, s.dquery.p, s.dkey.p,
                              s.core.p, s.recurrent.p, s.a.p, s.b.p, b.gates.p, s.gated.p, b.norm.p, s.z.p,
                              int32(c.key_heads), int32(c.value_heads), int32(c.key_dim), int32(c.value_dim),
                              int32(c.kernel), int32(t), int32(channels), c.eps};
                    a->check(a->delta_mixer(a->ctx, &d));
                } else {
                    a->op(ConvSilu, channels, {s.convolved.p, s.projected.p, b.conv.p, s.conv_state.p},
                          {c.kernel, t, channels, snapshot_rows}, {});
                    a->op(DeltaQk, vh * t, {s.dquery.p, s.convolved.p, s.dkey.p},
                          {c.key_heads, c.value_heads, c.key_dim, channels}, {});
                    int rule = DeltaRuleGated;
                    float *r5 = s.a.p, *r6 = s.b.p, *r7 = b.gates.p;
                    if (!a->runs(DeltaRuleGated)) {
                        a->op(DeltaGates, vh * t, {s.decay.p, s.a.p, s.b.p, b.dt.p, b.alog.p, s.beta.p}, {vh}, {});
                        rule = DeltaRule;
                        r5 = s.decay.p;
                        r6 = s.beta.p;
                        r7 = nullptr;
                    }
                    a->op(rule, vd, {s.core.p, s.dquery.p, s.dkey.p, s.convolved.p, s.recurrent.p, r5, r6, r7},
                          {c.key_dim, c.value_dim, c.key_heads, c.value_heads, t, channels, snapshot_rows}, {});
                    if (a->runs(RmsNormGate)) {
                        a->op(RmsNormGate, vh * t, {s.gated.p, s.core.p, b.norm.p, s.z.p}, {c.value_dim}, {c.eps, 0.f});
                    } else {
                        norm_op(s.core.p, b.norm, s.normalized.p, c.value_dim, vh * t, c.eps, 0.f);
                        a->op(SiluProduct, vd * t, {s.gated.p, s.z.p, s.normalized.p}, {}, {});
                    }
                }
                post_normed = project_norm(b.out, s.gated, mixed, residual, x, mixed, b.post, b.eps);
            }
            record(layer, "mixed", mixed, h);
            if (!post_normed) add_norm(residual.p, x.p, mixed.p, b.post, norm.p, b.eps);
            record(layer, "after_mixer", residual, h);
            record(layer, "post_norm", norm, h);
            // GLU choice (src/device.rs:2153-2196), with the fp32 arm.
            Api::Glu glu = (b.gate.bf16 && b.up.bf16)   ? a->glu_bf16
                           : (b.gate.int8 && b.up.int8) ? a->glu_i8
                           : (b.gate.f32() && b.up.f32()) ? a->glu_f32
                                                          : nullptr;
            if (glu && b.gate.rows == b.up.rows && b.gate.cols == b.up.cols) {
                require(norm.len >= t * h && b.gate.cols == h && product.len >= t * i_size && gate.len >= t * i_size &&
                            up.len >= t * i_size && b.gate.rows == i_size,
                        "device GLU shape");
                a->check(glu(a->ctx, product.p, gate.p, up.p, b.gate.buffer.p, b.up.buffer.p, norm.p, int32(i_size),
                             int32(h), int32(t)));
            } else {
                project_all(a, norm, {{&b.gate, &gate}, {&b.up, &up}}, t);
                a->op(SiluProduct, i_size * t, {product.p, gate.p, up.p}, {}, {});
            }
            record(layer, "ffn_product", product, i_size);
            // Edit overlay (src/device.rs:2198-2250): the product read back,
            // EditManifest::apply row by row, written back; after the down
            // projection the direction-removal correction is added.
            std::vector<float> correction;
            if (edited(layer)) {
                auto rows = product.read(t * i_size);
                for (size_t r = 0; r < t; ++r) {
                    auto c = apply_edit(layer, rows.data() + r * i_size);
                    correction.insert(correction.end(), c.begin(), c.end());
                }
                product.write(rows.data(), rows.size());
                record(layer, "ffn_intervened_product", product, i_size);
            }
            const bool last = layer + 1 == model->blocks.size();
            const DeviceBlock* next = (!last && fused_add_norm) ? &model->blocks[layer + 1] : nullptr;
            const Buffer& weight = last ? model->norm : model->blocks[layer + 1].input;
            const float eps = last ? cfg.rms_norm_eps : model->blocks[layer + 1].eps;
            bool down_normed;
            if ((next || last) && correction.empty())
                down_normed = project_norm(b.down, product, ffn, x, residual, ffn, weight, eps);
            else {
                b.down.project(product, ffn, t);
                down_normed = false;
            }
            if (!correction.empty()) {
                // `mixed` is free after the residual add above: the correction's staging
                mixed.write(correction.data(), correction.size());
                a->op(Add, h * t, {ffn.p, ffn.p, mixed.p}, {}, {});
            }
            record(layer, "ffn", ffn, h);
            normed = next != nullptr;
            if (down_normed) {
                final_normed = next == nullptr;
            } else if (next) {
                add_norm(x.p, residual.p, ffn.p, next->input, norm.p, next->eps);
            } else {
                a->op(Add, h * t, {x.p, residual.p, ffn.p}, {}, {});
            }
            record(layer, "output", x, h);
        }
        if (!final_normed) norm_op(x.at((t - 1) * h), model->norm, norm.p, h, 1, cfg.rms_norm_eps, 1.f);
        std::vector<float> out;
        const size_t vocab = size_t(cfg.vocab_size);
        if (logit_rows == 1) {
            model->output().project(norm, logits, 1);
            if (greedy_rows)
                pick_rows(1);
            else
                out = logits.read(vocab);
        } else if (logit_rows > 1) {
            norm_op(x.p, model->norm, norm.p, h, t, cfg.rms_norm_eps, 1.f);
            model->output().project(norm, logits, t);
            if (greedy_rows)
                pick_rows(t);
            else
                out = logits.read(t * vocab);
        }
        if (capture) {
            auto n = norm.read(h);
            rec->fn(rec->user, int(model->blocks.size()) - 1, "normalized", n.data(), int64_t(h));
            if (!out.empty()) rec->fn(rec->user, int(model->blocks.size()) - 1, "logits", out.data(), int64_t(vocab));
        }
        position += t;
        return out;
    }

    // inspect_state part sizes (src/device.rs:2380-2424)
    int64_t state_size(int layer, int which) const {
        require(layer >= 0 && size_t(layer) < model->blocks.size(), "layer out of range");
        const DeviceBlock& b = model->blocks[size_t(layer)];
        switch (which) {
        case 0: return b.attention ? 0 : int64_t(b.qkv.rows * (b.dc.kernel - 1));
        case 1: return b.attention ? 0 : int64_t(b.dc.value_heads * b.dc.key_dim * b.dc.value_dim);
        case 2:
        case 3: return b.attention ? int64_t(position * b.ac.kv_heads * b.ac.head_dim) : 0;
        }
        throw Error{"state part"};
    }
    const Buffer& state_buffer(int layer, int which) const {
        const MixerRun& m = mixers[size_t(layer)];
        switch (which) {
        case 0: return m.conv_state;
        case 1: return m.recurrent;
        case 2: return m.keys;
        default: return m.values;
        }
    }
};

extern "C" {

const char* qe_last_error(void) { return g_error.c_str(); }

QeModel* qe_model_load(const char* bridge_path, int expect_kind, const QwConfig* config, const float* const* tensors,
                       int format, int disable) {
    QeModel* out = nullptr;
    guarded([&] {
        auto m = std::make_unique<QeModel>();
        m->api = std::make_unique<Api>();
        m->api->open(bridge_path, expect_kind, disable);
        const Api* a = m->api.get();
        const QwConfig& c = *config;
        require(c.num_layers > 0 && c.num_layers <= QW_MAX_LAYERS && c.hidden_size > 0 && c.vocab_size > 0,
                "invalid config");
        m->config = c;
        m->info = a->info(a->ctx);
        const size_t H = size_t(c.hidden_size), I = size_t(c.intermediate_size);
        // upload (src/device.rs:978-1042)
        if (format == QE_INT8) {
            m->embedding = DeviceMatrix::make(a, tensors[0], size_t(c.vocab_size), H, QE_BF16_EXACT);
            m->lm_head = DeviceMatrix::make(a, tensors[0], size_t(c.vocab_size), H, QE_INT8);
        } else {
            m->embedding = DeviceMatrix::make(a, tensors[0], size_t(c.vocab_size), H, format);
        }
        m->norm = upload(a, tensors[1], H);
        const size_t channels = size_t(2 * c.key_heads * c.key_dim + c.value_heads * c.value_dim);
        for (int l = 0; l < c.num_layers; ++l) {
            const float* const* t = tensors + QW_SLOTS_BASE + size_t(l) * QW_SLOTS_LAYER;
            DeviceBlock b;
            b.attention = c.attention[l] != 0;
            b.eps = c.rms_norm_eps;
            if (b.attention) {
                b.ac = AttentionCfg{size_t(c.num_heads), size_t(c.num_kv_heads), size_t(c.head_dim),
                                    size_t(c.rotary_dim), c.rope_theta, c.rms_norm_eps};
                size_t d = b.ac.head_dim, q = b.ac.heads * d, kv = b.ac.kv_heads * d;
                b.q = DeviceMatrix::make(a, t[QW_Q], 2 * q, H, format);
                b.k = DeviceMatrix::make(a, t[QW_K], kv, H, format);
                b.v = DeviceMatrix::make(a, t[QW_V], kv, H, format);
                b.o = DeviceMatrix::make(a, t[QW_O], H, q, format);
                b.qn = upload(a, t[QW_Q_NORM], d);
                b.kn = upload(a, t[QW_K_NORM], d);
                std::vector<float> qkn(t[QW_Q_NORM], t[QW_Q_NORM] + d);
                qkn.insert(qkn.end(), t[QW_K_NORM], t[QW_K_NORM] + d);
                b.qkn = upload(a, qkn.data(), qkn.size());
            } else {
                b.dc = DeltaCfg{size_t(c.key_heads), size_t(c.value_heads), size_t(c.key_dim), size_t(c.value_dim),
                                size_t(c.conv_kernel), c.rms_norm_eps};
                size_t vd = b.dc.value_heads * b.dc.value_dim, vh = b.dc.value_heads;
                b.qkv = DeviceMatrix::make(a, t[QW_QKV], channels, H, format);
                b.z = DeviceMatrix::make(a, t[QW_Z], vd, H, format);
                b.a = DeviceMatrix::make(a, t[QW_A], vh, H, format);
                b.b = DeviceMatrix::make(a, t[QW_B], vh, H, format);
                b.conv = upload(a, t[QW_CONV], channels * b.dc.kernel);
                b.dt = upload(a, t[QW_DT], vh);
                b.alog = upload(a, t[QW_A_LOG], vh);
                std::vector<float> gates(t[QW_DT], t[QW_DT] + vh);
                gates.insert(gates.end(), t[QW_A_LOG], t[QW_A_LOG] + vh);
                b.gates = upload(a, gates.data(), gates.size());
                b.norm = upload(a, t[QW_DELTA_NORM], b.dc.value_dim);
                b.out = DeviceMatrix::make(a, t[QW_OUT], H, vd, format);
            }
            b.input = upload(a, t[QW_INPUT_NORM], H);
            b.post = upload(a, t[QW_POST_NORM], H);
            b.gate = DeviceMatrix::make(a, t[QW_GATE], I, H, format);
            b.up = DeviceMatrix::make(a, t[QW_UP], I, H, format);
            b.down = DeviceMatrix::make(a, t[QW_DOWN], H, I, format);
            // the prefill projections' planes (optional bridge symbols): every
            // fp32, BF16 or int8 block matrix of more than 16 rows with
            // 4-aligned columns (the a / b rows have a kernel of their own)
            for (const DeviceMatrix* dm : {&b.q, &b.k, &b.v, &b.o, &b.qkv, &b.z, &b.out, &b.gate, &b.up, &b.down}) {
                if (!dm->buffer.p || dm->rows <= 16 || dm->cols % 4 != 0) continue;
                if (dm->f32() && a->gemm_f32_prepare)
                    a->check(a->gemm_f32_prepare(a->ctx, dm->buffer.p, int32(dm->rows), int32(dm->cols)));
                else if (dm->bf16 && a->gemm_bf16_prepare)
                    a->check(a->gemm_bf16_prepare(a->ctx, dm->buffer.p, int32(dm->rows), int32(dm->cols)));
                else if (dm->int8 && a->gemm_i8_prepare)
                    a->check(a->gemm_i8_prepare(a->ctx, dm->buffer.p, int32(dm->rows), int32(dm->cols)));
            }
            m->blocks.push_back(std::move(b));
        }
        a->sync();
        out = m.release();
    });
    return out;
}

static void destroy_model(QeModel* m) {
    // Buffers free through the api: release them before the context goes.
    m->blocks.clear();
    m->embedding = DeviceMatrix{};
    m->lm_head.reset();
    m->norm = Buffer{};
    delete m;
}
void qe_model_free(QeModel* m) {
    if (!m) return;
    m->released = true;
    if (m->runs.load() == 0) destroy_model(m);
}

const char* qe_model_info(QeModel* m) { return m->info.c_str(); }

void qe_model_weight_summary(QeModel* m, int64_t* bf16, int64_t* matrices, int64_t* bytes) {
    std::vector<const DeviceMatrix*> all{&m->embedding};
    if (m->lm_head) all.push_back(&*m->lm_head);
    for (auto& b : m->blocks) {
        for (auto* x : {&b.gate, &b.up, &b.down}) all.push_back(x);
        if (b.attention)
            for (auto* x : {&b.q, &b.k, &b.v, &b.o}) all.push_back(x);
        else
            for (auto* x : {&b.qkv, &b.z, &b.a, &b.b, &b.out}) all.push_back(x);
    }
    int64_t nb = 0, total = 0;
    for (auto* x : all) {
        nb += x->bf16;
        total += int64_t(x->bytes());
    }
    *bf16 = nb;
    *matrices = int64_t(all.size());
    *bytes = total;
}

int qe_model_sync(QeModel* m) {
    return guarded([&] { m->api->sync(); });
}
int qe_model_profile(QeModel* m, int on) {
    return guarded([&] {
        require(m->api->profile != nullptr, "bridge has no profiler (qr_profile)");
        m->api->check(m->api->profile(m->api->ctx, on));
    });
}
long qe_model_profile_read(QeModel* m, char* out, size_t len) {
    if (!m->api->profile_read) {
        g_error = "bridge has no profiler (qr_profile_read)";
        return -1;
    }
    return m->api->profile_read(m->api->ctx, out, len);
}

void qe_model_set_run_budget(QeModel* m, uint64_t bytes) { m->run_budget = bytes; }
uint64_t qe_model_run_bytes(QeModel* m, int64_t capacity, int64_t chunk) {
    return m->run_bytes(size_t(capacity), std::min(size_t(chunk), size_t(capacity)));
}

QeRun* qe_run_new(QeModel* m, int64_t capacity, int64_t chunk, int64_t snapshots) {
    QeRun* out = nullptr;
    guarded([&] {
        require(capacity > 0 && chunk > 0 && snapshots >= 0, "run shape");
        if (snapshots > 0)
            require(m->api->snapshots && size_t(snapshots) < kVerifyRows,
                    "bridge has no state snapshots (qr_snapshots), or snapshots not 1..=7");
        auto r = std::make_unique<QeRun>();
        r->model = m;
        r->build(size_t(capacity), size_t(chunk), size_t(snapshots));
        out = r.release();
        ++m->runs;
    });
    return out;
}
void qe_run_free(QeRun* r) {
    if (!r) return;
    QeModel* m = r->model;
    delete r;  // its buffers go back through the model's bridge first
    if (m && --m->runs == 0 && m->released) destroy_model(m);
}

int qe_run_decode_plan(QeRun* r) { return r && r->plan ? 1 : 0; }

int qe_run_reset(QeRun* r) {
    return guarded([&] {
        QeRun fresh;
        fresh.model = r->model;
        fresh.build(r->capacity, r->chunk, r->snapshots);
        r->mixers = std::move(fresh.mixers);
        r->x = std::move(fresh.x);
        r->norm = std::move(fresh.norm);
        r->mixed = std::move(fresh.mixed);
        r->residual = std::move(fresh.residual);
        r->gate = std::move(fresh.gate);
        r->up = std::move(fresh.up);
        r->product = std::move(fresh.product);
        r->ffn = std::move(fresh.ffn);
        r->logits = std::move(fresh.logits);
        r->picks = std::move(fresh.picks);
        r->drop_plan();
        r->plan = fresh.plan;  // over the buffers moved in above
        fresh.plan = nullptr;
        r->position = 0;
        r->failed = false;
        r->pending.reset();
        r->snapshot_rows = 0;
        r->greedy_rows = false;
        r->picked.clear();
        r->pick_slot = 0;
        r->logits_unread = false;
    });
}

int64_t qe_run_position(QeRun* r) { return int64_t(r->position); }

int qe_step(QeRun* r, uint32_t id, float* logits, qe_record_fn record, void* user) {
    return guarded([&] {
        Record rec{record, user};
        auto l = r->step(id, record ? &rec : nullptr);
        if (logits) std::memcpy(logits, l.data(), l.size() * 4);
    });
}

int qe_step_greedy(QeRun* r, uint32_t id, uint32_t* next) {
    return guarded([&] { *next = r->step_greedy(id); });
}

int qe_prefill(QeRun* r, const uint32_t* ids, int64_t n, float* last_logits, int* has_logits) {
    return guarded([&] {
        require(n >= 0, "negative length");
        auto l = r->prefill(ids, size_t(n));
        if (has_logits) *has_logits = l.has_value();
        if (l && last_logits) std::memcpy(last_logits, l->data(), l->size() * 4);
    });
}

int qe_verify(QeRun* r, const uint32_t* ids, int64_t n, float* logits) {
    return guarded([&] {
        auto l = r->verify(ids, size_t(n));
        if (logits) std::memcpy(logits, l.data(), l.size() * 4);
    });
}
int qe_verify_rollback(QeRun* r, const uint32_t* ids, int64_t n, float* logits) {
    return guarded([&] {
        auto l = r->verify_rollback(ids, size_t(n));
        if (logits) std::memcpy(logits, l.data(), l.size() * 4);
    });
}
int qe_verify_rollback_greedy(QeRun* r, const uint32_t* ids, int64_t n, uint32_t* picks) {
    return guarded([&] {
        auto p = r->verify_rollback_greedy(ids, size_t(n));
        std::memcpy(picks, p.data(), p.size() * 4);
    });
}
int qe_accept(QeRun* r, int64_t rows) {
    return guarded([&] { r->accept(size_t(rows)); });
}
int qe_unread_logits(QeRun* r, float* logits) {
    int have = 0;
    int s = guarded([&] {
        if (!r->logits_unread) return;
        auto l = r->logits.read(size_t(r->model->config.vocab_size));
        std::memcpy(logits, l.data(), l.size() * 4);
        have = 1;
    });
    return s ? -1 : have;
}

int64_t qe_state_size(QeRun* r, int layer, int which) {
    int64_t n = -1;
    guarded([&] { n = r->state_size(layer, which); });
    return n;
}
int qe_state_read(QeRun* r, int layer, int which, float* out) {
    return guarded([&] {
        require(!r->failed, "cannot inspect poisoned device state");
        int64_t n = r->state_size(layer, which);
        if (n <= 0) return;
        auto v = r->state_buffer(layer, which).read(size_t(n));
        std::memcpy(out, v.data(), size_t(n) * 4);
    });
}
int qe_state_write(QeRun* r, int layer, int which, const float* values, int64_t n) {
    return guarded([&] {
        require(!r->failed, "device state does not fit this run");
        require(n >= 0, "negative length");
        if (n == 0) return;
        const Buffer& b = r->state_buffer(layer, which);
        require_finite(values, size_t(n));
        b.write(values, size_t(n));
    });
}
int qe_state_set_position(QeRun* r, int64_t position) {
    return guarded([&] {
        require(position >= 0 && size_t(position) <= r->capacity, "position beyond capacity");
        r->position = size_t(position);
        r->logits_unread = false;
    });
}

QeCheckpoint* qe_checkpoint(QeRun* r) {
    QeCheckpoint* out = nullptr;
    guarded([&] {
        require(!r->failed, "cannot checkpoint poisoned device state");
        auto c = std::make_unique<QeCheckpoint>();
        c->position = r->position;
        for (size_t l = 0; l < r->model->blocks.size(); ++l) {
            const DeviceBlock& b = r->model->blocks[l];
            if (b.attention) {
                c->delta.emplace_back(std::nullopt);
                continue;
            }
            std::vector<float> conv;
            if (b.dc.kernel > 1) conv = r->mixers[l].conv_state.read(b.qkv.rows * (b.dc.kernel - 1));
            auto rec = r->mixers[l].recurrent.read(b.dc.value_heads * b.dc.key_dim * b.dc.value_dim);
            c->delta.emplace_back(std::make_pair(std::move(conv), std::move(rec)));
        }
        out = c.release();
    });
    return out;
}
QeCheckpoint* qe_initial_checkpoint(QeRun* r) {
    auto c = new QeCheckpoint;
    for (auto& b : r->model->blocks) {
        if (b.attention)
            c->delta.emplace_back(std::nullopt);
        else
            c->delta.emplace_back(std::make_pair(std::vector<float>(b.qkv.rows * (b.dc.kernel - 1), 0.f),
                                                 std::vector<float>(b.dc.value_heads * b.dc.key_dim * b.dc.value_dim, 0.f)));
    }
    return c;
}
int qe_restore(QeRun* r, const QeCheckpoint* c) {
    return guarded([&] {
        r->logits_unread = false;
        require(!r->failed && c->position <= r->position && c->delta.size() == r->mixers.size(),
                "device restore needs an earlier checkpoint of this run");
        for (size_t l = 0; l < c->delta.size(); ++l) {
            if (!c->delta[l]) continue;
            auto& [conv, rec] = *c->delta[l];
            if (!conv.empty()) r->mixers[l].conv_state.write(conv.data(), conv.size());
            r->mixers[l].recurrent.write(rec.data(), rec.size());
        }
        r->position = c->position;
    });
}
void qe_checkpoint_free(QeCheckpoint* c) { delete c; }
int64_t qe_checkpoint_position(const QeCheckpoint* c) { return int64_t(c->position); }

// generate (src/device/speculative.rs:53-160), greedy, without the MTP
// head's hidden rows.
int qe_speculative_generate(QeRun* r, const QeDraft* draft, const uint32_t* prompt, int64_t n_prompt,
                            int64_t max_new, int64_t depth, const uint32_t* eos, int64_t n_eos, uint32_t* out,
                            int64_t* n_out, QeSpecStats* stats) {
    return guarded([&] {
        require(draft && draft->absorb && draft->draft && out && n_out, "speculative: missing draft or output");
        require(n_prompt > 0 && depth >= 1 && depth <= 7 && size_t(depth) <= r->snapshots && r->position == 0,
                "speculative: empty prompt, depth beyond the run's snapshots, or used run");
        using clock = std::chrono::steady_clock;
        auto secs = [](clock::time_point t) { return std::chrono::duration<double>(clock::now() - t).count(); };
        QeSpecStats st{};
        auto is_eos = [&](uint32_t id) { return std::find(eos, eos + std::max<int64_t>(n_eos, 0), id) != eos + std::max<int64_t>(n_eos, 0); };
        int64_t n = 0;
        *n_out = 0;
        // Empty drafts in a row: with no end-of-sequence token to stop at, the
        // next pass after one runs a burst of chained greedy steps (2, 4, then
        // 8 tokens) instead of one verify row, and the draft absorbs them all;
        // the output is the same greedy sequence, with fewer host reads.
        int64_t empty = 0;
        constexpr int64_t kMaxBurst = 8;
        if (max_new > 0) {
            auto t = clock::now();
            auto logits = r->prefill(prompt, size_t(n_prompt));
            require(logits.has_value(), "speculative: prefill returned no logits");
            st.prefill_s = secs(t);
            uint32_t cur = QeRun::select_greedy(*logits);
            out[n++] = cur;
            // the draft absorbs the true next token of every prompt position
            std::vector<uint32_t> next(prompt + 1, prompt + n_prompt);
            next.push_back(cur);
            t = clock::now();
            require(draft->absorb(draft->user, next.data(), int64_t(next.size())) == 0, "speculative: draft absorb failed");
            st.draft_s += secs(t);
            while (!is_eos(cur) && n < max_new) {
                // a pass emits up to k + 1 tokens and needs k + 1 positions
                const int64_t room = std::min<int64_t>(max_new - n, int64_t(r->capacity - r->position));
                require(room > 0, "speculative: run capacity exhausted");
                const int64_t k = std::min<int64_t>(depth, room - 1);
                std::vector<uint32_t> rows(size_t(k) + 1);
                rows[0] = cur;
                t = clock::now();
                const int64_t got = k > 0 ? draft->draft(draft->user, k, rows.data() + 1) : 0;
                st.draft_s += secs(t);
                require(got >= 0 && got <= k, "speculative: draft failed");
                const int64_t burst = n_eos > 0 || got > 0 ? 1 : std::min<int64_t>(kMaxBurst, int64_t(1) << std::min<int64_t>(empty, 3));
                empty = got > 0 ? 0 : empty + 1;
                if (burst > 1 && std::min(burst, room) > 1 && r->can_chain()) {
                    const int64_t b = std::min(burst, room);
                    std::vector<uint32_t> emitted(static_cast<size_t>(b));
                    t = clock::now();
                    r->chained_greedy(cur, size_t(b), emitted.data());
                    st.verify_s += secs(t);
                    st.passes += 1;
                    t = clock::now();
                    require(draft->absorb(draft->user, emitted.data(), int64_t(emitted.size())) == 0,
                            "speculative: draft absorb failed");
                    st.draft_s += secs(t);
                    for (uint32_t id : emitted) {
                        out[n++] = id;
                        cur = id;
                    }
                    continue;
                }
                for (int64_t j = 1; j <= got; ++j)
                    require(rows[size_t(j)] < uint32_t(r->model->config.vocab_size), "speculative: draft token out of range");
                rows.resize(size_t(got) + 1);
                t = clock::now();
                const auto picks = r->verify_rollback_greedy(rows.data(), rows.size());
                std::vector<uint32_t> emitted;
                for (int64_t j = 0; j < got; ++j) st.offered[j] += 1;
                for (size_t j = 0; j < picks.size(); ++j) {
                    emitted.push_back(picks[j]);
                    if (j == size_t(got) || picks[j] != rows[j + 1]) break;
                    st.accepted[j] += 1;
                    if (is_eos(picks[j])) break;
                }
                r->accept(emitted.size());
                st.verify_s += secs(t);
                st.passes += 1;
                t = clock::now();
                require(draft->absorb(draft->user, emitted.data(), int64_t(emitted.size())) == 0,
                        "speculative: draft absorb failed");
                st.draft_s += secs(t);
                for (uint32_t id : emitted) {
                    out[n++] = id;
                    cur = id;
                    if (is_eos(id) || n >= max_new) break;
                }
            }
        }
        *n_out = n;
        if (stats) *stats = st;
    });
}

namespace {
// Prompt-lookup drafting over the token history.
struct NgramDraft {
    QeDraft api{};
    size_t max_ngram = 3;
    std::vector<uint32_t> history;
};
int ngram_absorb(void* user, const uint32_t* next, int64_t n) {
    auto* d = static_cast<NgramDraft*>(user);
    if (n < 0 || (n > 0 && !next)) return -1;
    // the history is the prompt's first token (never "next") plus every true next token
    d->history.insert(d->history.end(), next, next + n);
    return 0;
}
int64_t ngram_draft(void* user, int64_t k, uint32_t* out) {
    auto* d = static_cast<NgramDraft*>(user);
    const auto& h = d->history;
    for (size_t len = std::min(d->max_ngram, h.size() > 0 ? h.size() - 1 : 0); len >= 1; --len) {
        const uint32_t* tail = h.data() + h.size() - len;
        // the most recent earlier occurrence with k tokens after it, else the
        // one with the longest continuation
        size_t best_from = 0;
        int64_t best = 0;
        for (size_t start = h.size() - len; start-- > 0 && best < k;) {
            if (std::equal(tail, tail + len, h.data() + start)) {
                const size_t from = start + len;
                const int64_t m = std::min<int64_t>(k, int64_t(h.size() - from));
                if (m > best) {
                    best = m;
                    best_from = from;
                }
            }
        }
        if (best > 0) {
            std::copy(h.begin() + long(best_from), h.begin() + long(best_from) + best, out);
            return best;
        }
    }
    return 0;
}
}  // namespace

QeDraft* qe_draft_ngram_new(int64_t max_ngram) {
    auto* d = new NgramDraft;
    d->max_ngram = size_t(std::max<int64_t>(1, max_ngram));
    d->api = QeDraft{d, ngram_absorb, ngram_draft};
    return &d->api;
}
void qe_draft_ngram_free(QeDraft* d) {
    if (d) delete static_cast<NgramDraft*>(d->user);
}

// set_edit (src/device.rs:1401-1438) with EditManifest::validate
// (src/edit.rs:19-58), without the model revision (the engine loads tensors,
// not a checkpoint with a revision).
int qe_run_set_edit(QeRun* r, const QeEdit* edits, int64_t n, const float* const* tensors) {
    return guarded([&] {
        const QwConfig& c = r->model->config;
        if (n <= 0 || !edits) {
            r->edits.clear();
            r->edit_down.clear();
            return;
        }
        const size_t h = size_t(c.hidden_size), i_size = size_t(c.intermediate_size);
        std::vector<QeRun::EditEntry> out;
        std::vector<std::vector<float>> down(size_t(c.num_layers));
        for (int64_t k = 0; k < n; ++k) {
            const QeEdit& e = edits[k];
            require(e.layer >= 0 && e.layer < c.num_layers && e.tensor_name &&
                        std::string(e.tensor_name) ==
                            "model.language_model.layers." + std::to_string(e.layer) + ".mlp.down_proj.weight",
                    "edit target mismatch");
            require(e.n_columns > 0 && e.columns && std::isfinite(e.coefficient), "invalid edit columns/coefficient");
            std::vector<size_t> cols;
            for (int64_t j = 0; j < e.n_columns; ++j) {
                require(e.columns[j] >= 0 && size_t(e.columns[j]) < i_size, "invalid edit columns/coefficient");
                cols.push_back(size_t(e.columns[j]));
            }
            std::vector<size_t> unique = cols;
            std::sort(unique.begin(), unique.end());
            require(std::adjacent_find(unique.begin(), unique.end()) == unique.end(), "duplicate edit column");
            std::vector<float> dir;
            if (e.direction) {
                dir.assign(e.direction, e.direction + h);
                float norm = -0.f;
                for (float v : dir) {
                    require(std::isfinite(v), "NaN/Inf detected");
                    norm += v * v;
                }
                require(std::isfinite(norm) && norm > 0.f, "invalid direction norm");
            }
            out.push_back(QeRun::EditEntry{size_t(e.layer), cols, dir, e.coefficient});
            if (down[size_t(e.layer)].empty()) {
                const float* w = tensors ? tensors[QW_SLOTS_BASE + e.layer * QW_SLOTS_LAYER + QW_DOWN] : nullptr;
                require(w != nullptr, "edit needs the down matrix of every edited layer");
                down[size_t(e.layer)].assign(w, w + h * i_size);
            }
        }
        r->edits = std::move(out);
        r->edit_down = std::move(down);
    });
}

int qe_decode_greedy(QeRun* r, uint32_t first, int64_t n_new, uint32_t* ids, double* seconds) {
    return guarded([&] {
        double total = 0;
        uint32_t token = first;
        // the planned steps of step_greedy (forward's one-launch conditions),
        // queued back to back with one read-back
        if (n_new > 1 && r->can_chain()) {
            ids[0] = first;
            total = r->chained_greedy(first, size_t(n_new - 1), ids + 1);
            if (seconds) *seconds = total;
            return;
        }
        for (int64_t i = 0; i < n_new; ++i) {
            ids[i] = token;
            if (i + 1 == n_new) break;
            require(r->position < r->capacity, "context limit");
            auto t0 = std::chrono::steady_clock::now();
            token = r->step_greedy(token);
            total += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        }
        if (seconds) *seconds = total;
    });
}

void qe_quantize_int8_rows(const float* w, int64_t rows, int64_t cols, float* scales, int8_t* q) {
    quantize_rows(w, size_t(rows), size_t(cols), scales, q);
}

}  // extern "C"
