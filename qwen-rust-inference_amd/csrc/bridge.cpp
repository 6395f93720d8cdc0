// The qr_* C ABI (version 3) of the MI355X bridge: context, memory, op
// dispatch and the projection entry points, over the gfx950 kernels of
// gemv.hip, gemm.hip, ops.hip, attention.hip and deltanet.hip. Declarations
// and the reference entry point each one replaces: include/qwen_bridge.h.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <new>
#include <string>
#include <vector>

#include "common.h"

struct Context {
    char error[256] = {};
    char info[512] = {};
    hipStream_t stream = nullptr;
    unsigned* ticket = nullptr;   // add-norm tail counter (kept 0 between launches)
    float* argmax_parts = nullptr;  // per-slice partials of the two-pass argmax
    size_t argmax_parts_len = 0;
    float* attn_parts = nullptr;  // split partials of decode attention
    size_t attn_parts_len = 0;
    float* rule_chunks = nullptr;  // per-(chunk, head) records of the chunked DeltaRule
    size_t rule_chunks_len = 0;
    float* gemm_work = nullptr;  // K-split partial sums of prefill GEMMs
    size_t gemm_work_len = 0;
    // Prepared matrices, by the matrix's device address, for the prefill
    // projections of gemm_p3.hip: the three P3 planes of an fp32 matrix
    // (qr_gemm_f32_prepare), or the one P1 plane of a packed BF16 matrix
    // (qr_gemm_bf16_prepare) or of an int8 matrix's values (qr_gemm_i8_prepare;
    // its row scales stay in the matrix); dropped when the matrix is freed or
    // written.
    struct Prepared {
        int rows, cols;
        __bf16* w3;
        int planes;  // 3 (fp32) or 1 (BF16, int8)
        qr::WeightType kind;
        // int8: the rows' scales (the matrix's first `rows` words)
        const float* scales;
        // the matrix's extent in 32-bit words
        size_t words() const {
            const size_t n = size_t(rows) * size_t(cols);
            return kind == qr::WeightType::F32 ? n : kind == qr::WeightType::BF16 ? (n + 1) / 2 : rows + (n + 3) / 4;
        }
    };
    std::map<const float*, Prepared> prepared;
    // Words of each qr_alloc allocation, so that qr_free drops the planes of
    // any prepared matrix inside the freed range, not only one at its start.
    std::map<const float*, size_t> allocs;
    // A prepared GLU's combined gate / up planes (p3_glu_interleave), made on
    // the pair's first prefill GLU, so both projections and the silu product
    // run as one kernel; dropped with either matrix's planes.
    struct GluPair {
        int rows, cols;
        __bf16* w3;
        int planes;
    };
    std::map<std::pair<const float*, const float*>, GluPair> glu_pairs;
    // The P3 planes of a projection's input (xp), and a second buffer the GLU
    // writes its product's planes into while it reads xp (then they swap).
    __bf16* xp = nullptr;
    __bf16* xp_alt = nullptr;
    size_t xp_len = 0, xp_alt_len = 0;  // in BF16 elements
    // A producer (a norm, or a GLU's product, over at least kPlanesMinBatch
    // rows of a width some prepared matrix takes) may leave its output's planes
    // in xp as it writes the output: they stand for xp_src (xp_rows x xp_cols)
    // during the very next bridge call only (serial == xp_serial + 1), so
    // nothing written in between can make them stale. Every entry point
    // advances the serial.
    const float* xp_src = nullptr;
    int xp_rows = 0, xp_cols = 0;
    unsigned long serial = 0, xp_serial = 0;
    // The width of the projection that took the last RmsNormGate output right
    // after it (its rows span several groups), by group size: from then on such
    // a norm writes its planes in rows of that width.
    std::map<int, int> gate_width;
    // qr_set_option "decode_cooperative": one-launch decode plans made from
    // then on launch cooperatively (default: plain launches)
    bool decode_cooperative = false;
    // "decode_residency_check" (default 1): a plain-launched plan whose
    // blocks were not all resident at dispatch switches itself to
    // cooperative launches; "decode_residency_test" 1: every launch counts
    // as such (the switch exercised on an idle device)
    bool decode_residency_auto = true, decode_residency_test = false;
    const float* gate_out = nullptr;
    int gate_d = 0;
    unsigned long gate_serial = 0;
    // RoPE denominators theta^(2i / rot) per (theta bits, rot), device copies.
    std::map<std::pair<uint32_t, int>, float*> rope;
    // Profiler (qr_profile / QWEN_ROCM_PROFILE=1): a hipEvent pair on the
    // context stream around every bridge call, summed per label.
    bool profile = false, print_at_exit = false;
    struct Timed {
        std::string label;
        hipEvent_t start, stop;
    };
    std::vector<Timed> timed;
    std::vector<hipEvent_t> spare;
    std::map<std::string, std::pair<long, double>> totals;  // label -> (calls, ms)
};

namespace {

int fail(Context* c, const char* what, int status) {
    std::snprintf(c->error, sizeof(c->error), "%s status=%d (%s)", what, status,
                  status > 0 ? hipGetErrorString(hipError_t(status)) : "invalid argument");
    return status ? status : -1;
}
int launched(Context* c, const char* what, int status) { return status ? fail(c, what, status) : 0; }

hipEvent_t take_event(Context* c) {
    hipEvent_t e = nullptr;
    if (!c->spare.empty()) {
        e = c->spare.back();
        c->spare.pop_back();
    } else {
        (void)hipEventCreate(&e);
    }
    return e;
}
// Event pair around one bridge call when profiling; the label is built only then.
template <class L>
struct Scope {
    Context* c;
    hipEvent_t start = nullptr;
    std::string label;
    Scope(Context* ctx, L&& make) : c(ctx) {
        if (!c->profile) return;
        label = make();
        start = take_event(c);
        (void)hipEventRecord(start, c->stream);
    }
    ~Scope() {
        if (!start) return;
        hipEvent_t stop = take_event(c);
        (void)hipEventRecord(stop, c->stream);
        c->timed.push_back(Context::Timed{std::move(label), start, stop});
    }
};
template <class L>
Scope<L> scope(Context* c, L&& make) {
    return Scope<L>(c, std::forward<L>(make));
}
void collect(Context* c) {
    for (auto& t : c->timed) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, t.start, t.stop) == hipSuccess) {
            auto& v = c->totals[t.label];
            v.first += 1;
            v.second += ms;
        }
        c->spare.push_back(t.start);
        c->spare.push_back(t.stop);
    }
    c->timed.clear();
}
const char* wname(qr::WeightType t) {
    return t == qr::WeightType::F32 ? "f32" : t == qr::WeightType::BF16 ? "bf16" : "i8";
}
std::string shape(int rows, int cols, int batch) {
    return std::to_string(rows) + "x" + std::to_string(cols) + (batch > 1 ? " t" + std::to_string(batch) : "");
}
const char* op_name(int op) {
    static const char* names[] = {"?", "rms_norm", "add", "silu_product", "conv_silu", "delta_qk", "delta_gates",
                                  "delta_rule", "attention_query", "attention_kv", "attention_read", "embed_bf16",
                                  "add_rms_norm", "rms_norm_gate", "delta_rule_gated", "attention_query_kv", "argmax",
                                  "embed_bf16_picked"};
    return op >= 1 && op <= 17 ? names[op] : "?";
}

// Grows a bridge-owned scratch buffer (synchronising before a reallocation,
// since queued kernels may still use the old one).
int ensure(Context* c, float** buf, size_t* len, size_t need, const char* what) {
    if (need <= *len) return 0;
    if (*buf) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(*buf);
        *buf = nullptr;
        *len = 0;
    }
    auto st = hipMalloc(reinterpret_cast<void**>(buf), need * sizeof(float));
    if (st != hipSuccess) return fail(c, what, int(st));
    *len = need;
    return 0;
}

const void* i8_packed(const float* packed) { return packed; }

// ---- prepared fp32 and BF16 matrices (csrc/gemm_p3.hip)
// Projections of at least this many tokens take the P3 planes when their
// matrix is prepared (fewer tokens: the split-BF16 kernel, whose tiles the
// small batches fill as well).
constexpr int kPlanesMinBatch = 64;

// The prepared planes of matrix a of format t (fp32: three planes; BF16 and
// int8: one).
const Context::Prepared* prepared_for(Context* c, qr::WeightType t, const void* a, int rows, int cols, int batch) {
    if (batch < kPlanesMinBatch || rows <= 16) return nullptr;
    auto it = c->prepared.find(static_cast<const float*>(a));
    if (it == c->prepared.end() || it->second.rows != rows || it->second.cols != cols || it->second.kind != t)
        return nullptr;
    return &it->second;
}
// A planes buffer large enough for batch rows of cols (queued work on the old
// buffer drains first).
int grow_planes(Context* c, __bf16** buf, size_t* len, int cols, int batch) {
    const size_t need = qr::p3_elements(batch, cols);
    if (need <= *len) return 0;
    if (*buf) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(*buf);
        *buf = nullptr;
        *len = 0;
    }
    auto st = hipMalloc(reinterpret_cast<void**>(buf), need * sizeof(__bf16));
    if (st != hipSuccess) return fail(c, "hipMalloc split input", int(st));
    *len = need;
    return 0;
}
int grow_xp(Context* c, int cols, int batch) {
    if (qr::p3_elements(batch, cols) > c->xp_len) c->xp_src = nullptr;
    return grow_planes(c, &c->xp, &c->xp_len, cols, batch);
}
// x's P3 planes into c->xp: already there when the previous bridge call
// produced x with them, else split now.
int split_input(Context* c, const float* x, int cols, int batch) {
    if (c->gate_out == x && c->gate_serial + 1 == c->serial && cols % c->gate_d == 0)
        c->gate_width[c->gate_d] = cols;  // a gated norm's output projected: its row width
    if (c->xp_src == x && c->xp_rows == batch && c->xp_cols == cols && c->xp_serial + 1 == c->serial) return 0;
    c->xp_src = nullptr;
    if (int st = grow_xp(c, cols, batch)) return st;
    auto s = scope(c, [&] { return std::string("p3_split ") + shape(batch, cols, 1); });
    return launched(c, "p3_split", qr::p3_split(c->stream, c->xp, x, batch, cols));
}
// Whether a producer of `rows` rows of width `cols` should also write the
// planes: enough rows for the planes path and a prepared matrix of that width.
bool planes_wanted(Context* c, int cols, int rows) {
    if (rows < kPlanesMinBatch || !qr::p3_cols_ok(cols)) return false;
    for (auto& kv : c->prepared)
        if (kv.second.cols == cols && kv.second.rows > 16) return true;
    return false;
}
// Records that c->xp now holds src's planes (for the next bridge call).
void planes_made(Context* c, const float* src, int rows, int cols) {
    c->xp_src = src;
    c->xp_rows = rows;
    c->xp_cols = cols;
    c->xp_serial = c->serial;
}
int p3_project(Context* c, float* y, const Context::Prepared& p, int batch) {
    if (int st = ensure(c, &c->gemm_work, &c->gemm_work_len, qr::p3_gemm_scratch(batch, p.rows, p.cols, p.planes),
                        "hipMalloc GEMM split"))
        return st;
    auto s = scope(c, [&] {
        return std::string("gemm_") + wname(p.kind) + (p.planes == 3 ? "_p3 " : "_p1 ") + shape(p.rows, p.cols, batch);
    });
    return launched(c, "gemm_p3", qr::p3_gemm(c->stream, y, c->xp, p.w3, batch, p.rows, p.cols, c->gemm_work,
                                               c->gemm_work_len, p.planes, p.scales));
}
void drop_prepared(Context* c, std::map<const float*, Context::Prepared>::iterator it) {
    (void)hipStreamSynchronize(c->stream);  // queued GEMMs may still read the planes
    for (auto p = c->glu_pairs.begin(); p != c->glu_pairs.end();) {  // pairs holding a copy of them
        auto next = std::next(p);
        if (p->first.first == it->first || p->first.second == it->first) {
            (void)hipFree(p->second.w3);
            c->glu_pairs.erase(p);
        }
        p = next;
    }
    (void)hipFree(it->second.w3);
    c->prepared.erase(it);
}
// Drops the planes of every prepared matrix that [p, p + n) overlaps.
void invalidate_prepared(Context* c, const float* p, size_t n) {
    for (auto it = c->prepared.begin(); it != c->prepared.end();) {
        const float* a = it->first;
        const size_t len = it->second.words();
        auto next = std::next(it);
        if (p < a + len && a < p + n) drop_prepared(c, it);
        it = next;
    }
}

// The RoPE denominators of (theta, rot): powf(theta, float(2i) / float(rot)),
// the expression of the reference's rotate (src/attention.rs:49-50 and
// reference.h:41-47), evaluated by the host libm once per pair.
int rope_table(Context* c, float theta, int rot, const float** out) {
    uint32_t bits;
    std::memcpy(&bits, &theta, 4);
    auto key = std::make_pair(bits, rot);
    auto it = c->rope.find(key);
    if (it != c->rope.end()) {
        *out = it->second;
        return 0;
    }
    std::vector<float> host(size_t(rot / 2 > 0 ? rot / 2 : 1), 1.f);
    for (int i = 0; i < rot / 2; ++i) host[size_t(i)] = powf(theta, float(2 * i) / float(rot));
    float* dev = nullptr;
    auto st = hipMalloc(reinterpret_cast<void**>(&dev), host.size() * sizeof(float));
    if (st == hipSuccess)
        st = hipMemcpyAsync(dev, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice, c->stream);
    if (st == hipSuccess) st = hipStreamSynchronize(c->stream);
    if (st != hipSuccess) return fail(c, "RoPE table", int(st));
    c->rope[key] = dev;
    *out = dev;
    return 0;
}

int project(Context* c, qr::WeightType t, float* y, const void* a, const float* x, int rows, int cols, int batch) {
    if (rows < 1 || cols < 1 || batch < 1) return fail(c, "projection shape", -1);
    if (const Context::Prepared* p = prepared_for(c, t, a, rows, cols, batch)) {
        if (int st = split_input(c, x, cols, batch)) return st;
        return p3_project(c, y, *p, batch);
    }
    if (!qr::gemm_preferred(t, rows, cols, batch)) {
        auto s = scope(c, [&] { return std::string("gemv_") + wname(t) + " " + shape(rows, cols, batch); });
        qr::GemvItem it{y, a, rows};
        return launched(c, "gemv", qr::gemv_group(c->stream, t, &it, 1, x, cols, batch));
    }
    if (int st = ensure(c, &c->gemm_work, &c->gemm_work_len, qr::gemm_scratch(t, rows, cols, batch),
                        "hipMalloc GEMM split"))
        return st;
    auto s = scope(c, [&] { return std::string("gemm_") + wname(t) + " " + shape(rows, cols, batch); });
    return launched(c, "gemm", qr::gemm(c->stream, t, y, a, x, rows, cols, batch, c->gemm_work, c->gemm_work_len));
}

int group(Context* c, qr::WeightType t, int n, const QrProjection* items, const float* x, int cols, int batch) {
    if (n < 1 || cols < 1 || batch < 1) return fail(c, "GEMM group shape", -1);
    for (int i = 0; i < n; ++i)
        if (items[i].rows < 1) return fail(c, "GEMM group shape", -1);
    if (qr::gemm_preferred(t, items[0].rows, cols, batch)) {
        bool split = false;  // x's planes, made at the group's first prepared matrix
        for (int i = 0; i < n; ++i) {
            if (const Context::Prepared* p = prepared_for(c, t, items[i].a, items[i].rows, cols, batch)) {
                if (!split) {
                    if (int st = split_input(c, x, cols, batch)) return st;
                    split = true;
                }
                if (int st = p3_project(c, items[i].y, *p, batch)) return st;
                continue;
            }
            // two consecutive few-row fp32 or BF16 matrices (the DeltaNet a / b) in one launch
            if (i + 1 < n && qr::gemm_ab_ok(t, items[i].a, x, items[i].rows, cols, batch) &&
                qr::gemm_ab_ok(t, items[i + 1].a, x, items[i + 1].rows, cols, batch)) {
                auto sc = scope(c, [&] {
                    return std::string("gemm_") + wname(t) + "_ab " + shape(items[i].rows, cols, batch) + "+" +
                           shape(items[i + 1].rows, cols, batch);
                });
                if (int st = launched(c, "gemm_ab",
                                      qr::gemm_ab(c->stream, items[i].y, static_cast<const float*>(items[i].a),
                                                  items[i].rows, items[i + 1].y,
                                                  static_cast<const float*>(items[i + 1].a), items[i + 1].rows, x,
                                                  cols, batch, t)))
                    return st;
                ++i;
                continue;
            }
            if (int s = project(c, t, items[i].y, items[i].a, x, items[i].rows, cols, batch)) return s;
        }
        return 0;
    }
    qr::GemvItem its[64];
    if (n > 64) return fail(c, "GEMM group too large", -1);
    for (int i = 0; i < n; ++i) its[i] = qr::GemvItem{items[i].y, items[i].a, items[i].rows};
    auto s = scope(c, [&] {
        std::string l = std::string("gemv_") + wname(t) + "_group";
        for (int i = 0; i < n; ++i) l += (i ? "+" : " ") + shape(items[i].rows, cols, 1);
        return batch > 1 ? l + " t" + std::to_string(batch) : l;
    });
    return launched(c, "gemv_group", qr::gemv_group(c->stream, t, its, n, x, cols, batch));
}

int glu(Context* c, qr::WeightType t, float* product, float* gate_y, float* up_y, const float* gate, const float* up,
        const float* x, int rows, int cols, int batch) {
    if (rows < 1 || cols < 1 || batch < 1) return fail(c, "GLU shape", -1);
    if (!qr::gemm_preferred(t, rows, cols, batch)) {
        auto s = scope(c, [&] { return std::string("gemv_") + wname(t) + "_glu 2x" + shape(rows, cols, batch); });
        return launched(c, "gemv_glu", qr::gemv_glu(c->stream, t, product, gate, up, x, rows, cols, batch));
    }
    {
        const Context::Prepared* pg = prepared_for(c, t, gate, rows, cols, batch);
        const Context::Prepared* pu = prepared_for(c, t, up, rows, cols, batch);
        if (pg && pu && rows % 128 == 0) {
            // gate, up and the silu product as ONE kernel over the combined planes (gate_y / up_y
            // untouched, as the fused GLU), the product's planes for the next call (down)
            auto key = std::make_pair(gate, up);
            auto it = c->glu_pairs.find(key);
            if (it == c->glu_pairs.end()) {
                Context::GluPair pair{rows, cols, nullptr, pg->planes};
                const size_t elems = pg->planes == 3 ? qr::p3_elements(2 * rows, cols) : qr::p1_elements(2 * rows, cols);
                auto st = hipMalloc(reinterpret_cast<void**>(&pair.w3), elems * sizeof(__bf16));
                if (st != hipSuccess) return fail(c, "hipMalloc GLU planes", int(st));
                if (int e = qr::p3_glu_interleave(c->stream, pair.w3, pg->w3, pu->w3, rows, cols, pg->planes)) {
                    (void)hipStreamSynchronize(c->stream);
                    (void)hipFree(pair.w3);
                    return fail(c, "GLU planes", e);
                }
                it = c->glu_pairs.emplace(key, pair).first;
            }
            if (int st = split_input(c, x, cols, batch)) return st;
            if (int st = ensure(c, &c->gemm_work, &c->gemm_work_len,
                                qr::p3_glu_scratch(batch, rows, cols, it->second.planes), "hipMalloc GEMM split"))
                return st;
            const bool planes = planes_wanted(c, rows, batch);
            if (planes)
                if (int st = grow_planes(c, &c->xp_alt, &c->xp_alt_len, rows, batch)) return st;
            auto s = scope(c, [&] {
                return std::string("gemm_") + wname(t) + (it->second.planes == 3 ? "_p3_glu 2x" : "_p1_glu 2x") +
                       shape(rows, cols, batch);
            });
            const int st = qr::p3_gemm_glu(c->stream, product, planes ? c->xp_alt : nullptr, c->xp, it->second.w3,
                                           batch, rows, cols, c->gemm_work, c->gemm_work_len, it->second.planes,
                                           pg->scales, pu->scales);
            if (st == 0 && planes) {
                std::swap(c->xp, c->xp_alt);
                std::swap(c->xp_len, c->xp_alt_len);
                planes_made(c, product, batch, rows);
            }
            return launched(c, "gemm_p3_glu", st);
        }
        if (pg && pu) {  // gate and up into gate_y / up_y, then silu(gate_y) * up_y
            if (int st = split_input(c, x, cols, batch)) return st;
            if (int st = p3_project(c, gate_y, *pg, batch)) return st;
            if (int st = p3_project(c, up_y, *pu, batch)) return st;
            Params p{};
            p.p[0] = product;
            p.p[1] = gate_y;
            p.p[2] = up_y;
            auto s = scope(c, [&] { return std::string("silu_product ") + shape(rows, batch, 1); });
            return launched(c, "silu_product", qr::run_elementwise(c->stream, QR_SILU_PRODUCT, rows * batch, p));
        }
    }
    if (qr::gemm_glu_fused(t, gate, up, x, rows, cols, batch)) {  // gate_y / up_y untouched, as the reference's fused GLU
        auto s = scope(c, [&] { return std::string("gemm_") + wname(t) + "_glu 2x" + shape(rows, cols, batch); });
        return launched(c, "gemm_glu", qr::gemm_glu(c->stream, t, product, gate, up, x, rows, cols, batch));
    }
    if (int s = project(c, t, gate_y, gate, x, rows, cols, batch)) return s;
    if (int s = project(c, t, up_y, up, x, rows, cols, batch)) return s;
    Params p{};
    p.p[0] = product;
    p.p[1] = gate_y;
    p.p[2] = up_y;
    return launched(c, "silu_product", qr::run_elementwise(c->stream, QR_SILU_PRODUCT, rows * batch, p));
}

int add_norm(Context* c, qr::WeightType t, float* y, const void* a, const float* x, int rows, int cols,
             const QrAddNormPost* post) {
    if (rows < 1 || cols < 1 || !post) return fail(c, "GEMV+norm shape", -1);
    auto s = scope(c, [&] { return std::string("gemv_") + wname(t) + "_add_norm " + shape(rows, cols, 1); });
    return launched(c, "gemv_add_norm", qr::gemv_add_norm(c->stream, t, y, a, x, rows, cols, *post, c->ticket));
}

// Attention read of 2..8 rows: the decode path once per row over its own
// length, so every row equals the decode step of its position (the rows of a
// verify pass; reference native/rocm/bridge.cpp:197-215 does the same).
int attention_read(Context* c, int count, const Params& a) {
    const int rows = a.n[5] > 0 ? a.n[5] : 1;
    if (rows > 1 && rows <= 8) {
        const size_t q = size_t(a.n[0]) * size_t(a.n[1]);
        for (int r = 0; r < rows; ++r) {
            Params one = a;
            for (int slot : {0, 1, 4}) one.p[slot] = a.p[slot] + r * q;
            one.n[3] = a.n[3] + r;
            one.n[5] = 0;
            if (int s = attention_read(c, count, one)) return s;
        }
        return 0;
    }
    if (int s = ensure(c, &c->attn_parts, &c->attn_parts_len, qr::attention_scratch_needed(a), "hipMalloc attention"))
        return s;
    auto s = scope(c, [&] {
        return std::string(rows == 1 ? "attention_read decode len " : "attention_read prefill len ") +
               std::to_string(a.n[3]) + (rows > 1 ? " rows " + std::to_string(rows) : "");
    });
    return launched(c, "attention_read",
                    qr::run_attention_read(c->stream, count, a, c->attn_parts, c->attn_parts_len));
}

}  // namespace

extern "C" {

int qr_abi(void) { return 3; }
int qr_kind(void) { return QR_KIND_ROCM; }
int qr_max_op(void) { return QR_ATTENTION_QUERY_KV; }
int qr_snapshots(void) { return 1; }
int qr_argmax(void) { return 2; }

const char* qr_error(Context* c) { return c->error; }
const char* qr_info(Context* c) { return c->info; }

int qr_create(Context** out) {
    *out = nullptr;
    Context* c = new (std::nothrow) Context;
    if (!c) return -1;
    hipError_t h = hipSetDevice(0);
    if (h != hipSuccess) {
        delete c;
        return int(h);
    }
    h = hipStreamCreate(&c->stream);
    if (h != hipSuccess) {
        delete c;
        return int(h);
    }
    h = hipMalloc(reinterpret_cast<void**>(&c->ticket), 256);
    if (h == hipSuccess) h = hipMemset(c->ticket, 0, 256);
    if (h == hipSuccess) h = hipError_t(qr::argmax_fixed_init());  // qr_argmax_fixed's array on this device
    if (h != hipSuccess) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return int(h);
    }
    hipDeviceProp_t props{};
    int runtime = 0, driver = 0;
    auto ps = hipGetDeviceProperties(&props, 0);
    (void)hipRuntimeGetVersion(&runtime);
    (void)hipDriverGetVersion(&driver);
    std::snprintf(c->info, sizeof(c->info),
                  "device0=%s arch=%s cus=%d hbm_bytes=%zu l2_bytes=%d hip_runtime=%d driver_api=%d "
                  "bridge=qwen-mi355x gfx950 wave64",
                  ps == hipSuccess ? props.name : "unknown", ps == hipSuccess ? props.gcnArchName : "unknown",
                  ps == hipSuccess ? props.multiProcessorCount : 0, ps == hipSuccess ? size_t(props.totalGlobalMem) : 0,
                  ps == hipSuccess ? props.l2CacheSize : 0, runtime, driver);
    if (const char* p = std::getenv("QWEN_ROCM_PROFILE"))
        c->profile = c->print_at_exit = std::strcmp(p, "0") != 0 && p[0] != 0;
    *out = c;
    return 0;
}

int qr_set_option(Context* c, const char* name, int value) {
    ++c->serial;
    if (!name || (value != 0 && value != 1)) return fail(c, "unknown bridge option", -1);
    if (std::strcmp(name, "decode_cooperative") == 0) {  // this bridge's own: plans made after the call
        c->decode_cooperative = value != 0;
        return 0;
    }
    if (std::strcmp(name, "decode_residency_check") == 0) {
        c->decode_residency_auto = value != 0;
        return 0;
    }
    if (std::strcmp(name, "decode_residency_test") == 0) {
        c->decode_residency_test = value != 0;
        return 0;
    }
    if (std::strcmp(name, "attention_f16") != 0) return fail(c, "unknown bridge option", -1);
    if (value) return fail(c, "attention_f16 (16-bit prefill attention) is not offered: attention runs in fp32", -1);
    return 0;
}

int qr_sync(Context* c) {
    ++c->serial;
    auto s = hipStreamSynchronize(c->stream);
    if (s != hipSuccess) return fail(c, "hipStreamSynchronize", int(s));
    if (!c->timed.empty()) collect(c);
    return 0;
}

// Profiler switch (no counterpart in the reference's ABI; its bridge had the
// same event-pair profiler behind QWEN_ROCM_PROFILE, native/rocm/bridge.cpp:55-139).
int qr_profile(Context* c, int on) {
    ++c->serial;
    if (int s = qr_sync(c)) return s;
    c->profile = on != 0;
    if (on) c->totals.clear();
    return 0;
}

// Totals since qr_profile(c, 1) as text lines "calls<TAB>total_ms<TAB>label".
// Returns the length the full text needs (the text is truncated to `len`).
long qr_profile_read(Context* c, char* out, size_t len) {
    ++c->serial;
    if (qr_sync(c)) return -1;
    std::string text;
    for (auto& [label, v] : c->totals) {
        char line[64];
        std::snprintf(line, sizeof(line), "%ld\t%.6f\t", v.first, v.second);
        text += line + label + "\n";
    }
    if (out && len) {
        size_t n = text.size() < len - 1 ? text.size() : len - 1;
        std::memcpy(out, text.data(), n);
        out[n] = 0;
    }
    return long(text.size()) + 1;
}

void qr_destroy(Context* c) {
    if (!c) return;
    (void)hipStreamSynchronize(c->stream);
    if (c->print_at_exit) {
        collect(c);
        double all = 0;
        for (auto& [label, v] : c->totals) all += v.second;
        std::fprintf(stderr, "QWEN_ROCM_PROFILE: %.3f ms of GPU time in bridge calls\n%10s %12s %10s  %s\n", all,
                     "calls", "total_ms", "mean_us", "label");
        for (auto& [label, v] : c->totals)
            std::fprintf(stderr, "%10ld %12.3f %10.2f  %s\n", v.first, v.second, 1000 * v.second / double(v.first),
                         label.c_str());
    }
    for (auto& t : c->timed) {
        (void)hipEventDestroy(t.start);
        (void)hipEventDestroy(t.stop);
    }
    for (auto e : c->spare) (void)hipEventDestroy(e);
    for (auto& [key, dev] : c->rope) (void)hipFree(dev);
    if (c->ticket) (void)hipFree(c->ticket);
    if (c->argmax_parts) (void)hipFree(c->argmax_parts);
    if (c->attn_parts) (void)hipFree(c->attn_parts);
    if (c->rule_chunks) (void)hipFree(c->rule_chunks);
    if (c->gemm_work) (void)hipFree(c->gemm_work);
    for (auto& kv : c->prepared) (void)hipFree(kv.second.w3);
    for (auto& kv : c->glu_pairs) (void)hipFree(kv.second.w3);
    if (c->xp) (void)hipFree(c->xp);
    if (c->xp_alt) (void)hipFree(c->xp_alt);
    (void)hipStreamDestroy(c->stream);
    delete c;
}

int qr_alloc(Context* c, float** p, size_t n) {
    ++c->serial;
    if (n == 0) return fail(c, "empty allocation", -1);
    auto s = hipMalloc(reinterpret_cast<void**>(p), n * sizeof(float));
    if (s != hipSuccess) return fail(c, "hipMalloc", int(s));
    s = hipMemsetAsync(*p, 0, n * sizeof(float), c->stream);
    if (s != hipSuccess) {
        (void)hipFree(*p);
        *p = nullptr;
        return fail(c, "hipMemsetAsync", int(s));
    }
    c->allocs[*p] = n;
    return 0;
}

void qr_free(Context* c, float* p) {
    ++c->serial;
    auto it = c->allocs.find(p);
    const size_t n = it != c->allocs.end() ? it->second : 1;
    if (it != c->allocs.end()) c->allocs.erase(it);
    if (!c->prepared.empty()) invalidate_prepared(c, p, n);
    (void)hipFree(p);
}

int qr_write(Context* c, float* p, const float* host, size_t n) {
    ++c->serial;
    if (!c->prepared.empty()) invalidate_prepared(c, p, n);
    auto s = hipMemcpyAsync(p, host, n * sizeof(float), hipMemcpyHostToDevice, c->stream);
    if (s != hipSuccess) return fail(c, "H2D", int(s));
    return qr_sync(c);  // the host slice may be gone after return
}

int qr_read(Context* c, float* host, const float* p, size_t n) {
    ++c->serial;
    auto s = hipMemcpyAsync(host, p, n * sizeof(float), hipMemcpyDeviceToHost, c->stream);
    if (s != hipSuccess) return fail(c, "D2H", int(s));
    return qr_sync(c);
}

int qr_copy(Context* c, float* dest, const float* src, size_t n) {
    ++c->serial;
    if (!c->prepared.empty()) invalidate_prepared(c, dest, n);
    auto sc = scope(c, [&] { return std::string("copy"); });
    auto s = hipMemcpyAsync(dest, src, n * sizeof(float), hipMemcpyDeviceToDevice, c->stream);
    return s == hipSuccess ? 0 : fail(c, "D2D", int(s));
}

int qr_run(Context* c, int op, int count, const Params* ap) {
    ++c->serial;
    if (op < QR_RMS_NORM || op > QR_EMBED_BF16_PICKED || count < 1 || !ap) return fail(c, "invalid kernel", -1);
    const Params& a = *ap;
    hipStream_t s = c->stream;
    if (op == QR_ATTENTION_READ) return attention_read(c, count, a);  // timed inside
    auto sc = scope(c, [&] { return std::string(op_name(op)); });
    switch (op) {
    case QR_RMS_NORM:
    case QR_ADD_RMS_NORM:
    case QR_RMS_NORM_GATE:
        if (a.n[0] < 1) return fail(c, "norm shape", -1);
        {
            // the output's planes too, in rows of the width its projection takes: d for the
            // norms of a residual row, the learned width for a gated norm (groups of heads)
            int width = a.n[0];
            if (op == QR_RMS_NORM_GATE) {
                auto it = c->gate_width.find(a.n[0]);
                width = it == c->gate_width.end() ? 0 : it->second;
                c->gate_out = a.p[0];
                c->gate_d = a.n[0];
                c->gate_serial = c->serial;
            }
            const long total = long(count) * a.n[0];
            if (width > 0 && total % width == 0 && planes_wanted(c, width, int(total / width))) {
                const int rows = int(total / width);
                if (int st = grow_xp(c, width, rows)) return st;
                const int st = qr::run_rms_family_planes(s, op, count, a, c->xp, width);
                if (st == 0) {
                    planes_made(c, op == QR_ADD_RMS_NORM ? a.p[3] : a.p[0], rows, width);
                    return launched(c, "rms_norm", 0);
                }
                if (st != int(hipErrorNotSupported)) return launched(c, "rms_norm", st);
            }
        }
        return launched(c, "rms_norm", qr::run_rms_family(s, op, count, a));
    case QR_ADD:
    case QR_SILU_PRODUCT:
    case QR_DELTA_GATES:
    case QR_EMBED_BF16:
    case QR_EMBED_BF16_PICKED: return launched(c, "elementwise", qr::run_elementwise(s, op, count, a));
    case QR_CONV_SILU: return launched(c, "conv_silu", qr::run_conv_silu(s, count, a));
    case QR_DELTA_QK:
        if (a.n[0] < 1 || a.n[1] < 1 || a.n[1] % a.n[0] != 0) return fail(c, "DeltaQk heads", -1);
        return launched(c, "delta_qk", qr::run_delta_qk(s, count, a));
    case QR_DELTA_RULE:
    case QR_DELTA_RULE_GATED:
        if (a.n[0] < 1 || a.n[1] < 1 || a.n[0] > 256) return fail(c, "DeltaRule key_dim must be 1..256", -1);
        if (qr::delta_rule_chunked_ok(a, count)) {
            if (int st = ensure(c, &c->rule_chunks, &c->rule_chunks_len, qr::delta_rule_chunked_scratch(a),
                                "hipMalloc delta rule chunks"))
                return st;
            return launched(c, "delta_rule_chunked", qr::run_delta_rule_chunked(s, op == QR_DELTA_RULE_GATED, a,
                                                                                  c->rule_chunks, c->rule_chunks_len));
        }
        return launched(c, "delta_rule", qr::run_delta_rule(s, op == QR_DELTA_RULE_GATED, count, a));
    case QR_ATTENTION_QUERY:
    case QR_ATTENTION_KV:
    case QR_ATTENTION_QUERY_KV: {
        const float* denom = nullptr;
        if (int st = rope_table(c, a.f[1], a.n[1], &denom)) return st;
        return launched(c, "attention_qkv", qr::run_attention_qkv(s, op, count, a, denom));
    }
    case QR_ATTENTION_READ: return attention_read(c, count, a);
    case QR_ARGMAX: {
        if (a.n[0] < 1) return fail(c, "argmax shape", -1);
        if (int st = ensure(c, &c->argmax_parts, &c->argmax_parts_len, qr::argmax_parts_needed(count, a.n[0]),
                            "hipMalloc argmax"))
            return st;
        return launched(c, "argmax", qr::run_argmax(s, count, a, c->argmax_parts, c->argmax_parts_len));
    }
    }
    return fail(c, "invalid kernel", -1);
}

int qr_gemv(Context* c, float* y, const float* a, const float* x, int rows, int cols) {
    ++c->serial;
    return project(c, qr::WeightType::F32, y, a, x, rows, cols, 1);
}
int qr_gemm(Context* c, float* y, const float* a, const float* x, int rows, int cols, int batch) {
    ++c->serial;
    return project(c, qr::WeightType::F32, y, a, x, rows, cols, batch);
}
int qr_gemv_bf16(Context* c, float* y, const float* packed, const float* x, int rows, int cols) {
    ++c->serial;
    return project(c, qr::WeightType::BF16, y, packed, x, rows, cols, 1);
}
int qr_gemm_bf16(Context* c, float* y, const float* packed, const float* x, int rows, int cols, int batch) {
    ++c->serial;
    return project(c, qr::WeightType::BF16, y, packed, x, rows, cols, batch);
}
int qr_gemm_i8(Context* c, float* y, const float* packed, const float* x, int rows, int cols, int batch) {
    ++c->serial;
    return project(c, qr::WeightType::I8, y, i8_packed(packed), x, rows, cols, batch);
}

int qr_gemm_f32_group(Context* c, int n, const QrProjection* items, const float* x, int cols, int batch) {
    ++c->serial;
    return group(c, qr::WeightType::F32, n, items, x, cols, batch);
}
int qr_gemm_bf16_group(Context* c, int n, const QrProjection* items, const float* x, int cols, int batch) {
    ++c->serial;
    return group(c, qr::WeightType::BF16, n, items, x, cols, batch);
}
int qr_gemm_i8_group(Context* c, int n, const QrProjection* items, const float* x, int cols, int batch) {
    ++c->serial;
    return group(c, qr::WeightType::I8, n, items, x, cols, batch);
}

int qr_gemm_f32_glu(Context* c, float* product, float* gate_y, float* up_y, const float* gate, const float* up,
                    const float* x, int rows, int cols, int batch) {
    ++c->serial;
    return glu(c, qr::WeightType::F32, product, gate_y, up_y, gate, up, x, rows, cols, batch);
}
int qr_gemm_f32_prepare(Context* c, const float* a, int rows, int cols) {
    ++c->serial;
    if (!a || rows < 1 || cols < 1 || reinterpret_cast<uintptr_t>(a) % 16 != 0)
        return fail(c, "GEMM prepare shape", -1);
    if (!qr::p3_cols_ok(cols)) return 0;  // no planes: its projections keep the split-BF16 kernel
    auto it = c->prepared.find(a);
    if (it != c->prepared.end()) {
        if (it->second.rows == rows && it->second.cols == cols) return 0;
        drop_prepared(c, it);
    }
    __bf16* w3 = nullptr;
    auto st = hipMalloc(reinterpret_cast<void**>(&w3), qr::p3_elements(rows, cols) * sizeof(__bf16));
    if (st != hipSuccess) return fail(c, "hipMalloc GEMM planes", int(st));
    if (int e = qr::p3_split(c->stream, w3, a, rows, cols)) {
        (void)hipFree(w3);
        return fail(c, "p3_split", e);
    }
    c->prepared[a] = Context::Prepared{rows, cols, w3, 3, qr::WeightType::F32, nullptr};
    return 0;
}
// The one plane of a BF16 or int8 matrix (qr_gemm_bf16_prepare / qr_gemm_i8_prepare).
static int prepare_p1(Context* c, qr::WeightType t, const float* packed, int rows, int cols) {
    ++c->serial;
    if (!packed || rows < 1 || cols < 1 || reinterpret_cast<uintptr_t>(packed) % 16 != 0)
        return fail(c, "GEMM prepare shape", -1);
    // no plane (its projections keep the split-BF16 kernel) for other widths, and for int8
    // values that the odd count of scales before them leaves off 8-byte alignment
    if (!qr::p3_cols_ok(cols) || (t == qr::WeightType::I8 && rows % 2 != 0)) return 0;
    auto it = c->prepared.find(packed);
    if (it != c->prepared.end()) {
        if (it->second.rows == rows && it->second.cols == cols && it->second.kind == t) return 0;
        drop_prepared(c, it);
    }
    __bf16* w1 = nullptr;
    auto st = hipMalloc(reinterpret_cast<void**>(&w1), qr::p1_elements(rows, cols) * sizeof(__bf16));
    if (st != hipSuccess) return fail(c, "hipMalloc GEMM plane", int(st));
    const int e = t == qr::WeightType::BF16 ? qr::p1_from_bf16(c->stream, w1, packed, rows, cols)
                                            : qr::p1_from_i8(c->stream, w1, packed, rows, cols);
    if (e) {
        (void)hipFree(w1);
        return fail(c, "GEMM plane", e);
    }
    c->prepared[packed] =
        Context::Prepared{rows, cols, w1, 1, t, t == qr::WeightType::I8 ? packed : nullptr};
    return 0;
}
int qr_gemm_bf16_prepare(Context* c, const float* packed, int rows, int cols) {
    return prepare_p1(c, qr::WeightType::BF16, packed, rows, cols);
}
int qr_gemm_i8_prepare(Context* c, const float* packed, int rows, int cols) {
    return prepare_p1(c, qr::WeightType::I8, packed, rows, cols);
}
int qr_gemm_f32_release(Context* c, const float* a) {
    ++c->serial;
    auto it = c->prepared.find(a);
    if (it != c->prepared.end()) drop_prepared(c, it);
    return 0;
}
int qr_gemm_bf16_glu(Context* c, float* product, float* gate_y, float* up_y, const float* gate, const float* up,
                     const float* x, int rows, int cols, int batch) {
    ++c->serial;
    return glu(c, qr::WeightType::BF16, product, gate_y, up_y, gate, up, x, rows, cols, batch);
}
int qr_gemm_i8_glu(Context* c, float* product, float* gate_y, float* up_y, const float* gate, const float* up,
                   const float* x, int rows, int cols, int batch) {
    ++c->serial;
    return glu(c, qr::WeightType::I8, product, gate_y, up_y, gate, up, x, rows, cols, batch);
}

int qr_gemm_f32_add_norm(Context* c, float* y, const float* a, const float* x, int rows, int cols,
                         const QrAddNormPost* post) {
    ++c->serial;
    return add_norm(c, qr::WeightType::F32, y, a, x, rows, cols, post);
}
int qr_gemm_bf16_add_norm(Context* c, float* y, const float* packed, const float* x, int rows, int cols,
                          const QrAddNormPost* post) {
    ++c->serial;
    return add_norm(c, qr::WeightType::BF16, y, packed, x, rows, cols, post);
}
int qr_gemm_i8_add_norm(Context* c, float* y, const float* packed, const float* x, int rows, int cols,
                        const QrAddNormPost* post) {
    ++c->serial;
    return add_norm(c, qr::WeightType::I8, y, packed, x, rows, cols, post);
}

int qr_delta_mixer(Context* c, const QrDelta* d) {
    ++c->serial;
    if (!d || d->tokens < 1 || d->value_heads < 1 || d->key_heads < 1 || d->value_heads % d->key_heads != 0)
        return fail(c, "delta mixer shape", -1);
    if (qr::delta_mixer_decode_ok(*d)) {
        auto sc = scope(c, [&] { return std::string("delta_mixer decode"); });
        return launched(c, "delta_mixer", qr::delta_mixer_decode(c->stream, *d));
    }
    // Otherwise the four ops with the slots the engine gives them
    // (reference native/rocm/bridge.cpp:743-761), DeltaQk inside the chunked
    // rule at prefill lengths.
    const int vh = d->value_heads, vd = vh * d->value_dim, t = d->tokens;
    Params conv{}, qk{}, rule{}, gate{};
    conv.p[0] = d->convolved;
    conv.p[1] = const_cast<float*>(d->projected);
    conv.p[2] = const_cast<float*>(d->conv_w);
    conv.p[3] = d->conv_state;
    conv.n[0] = d->kernel;
    conv.n[1] = t;
    conv.n[2] = d->channels;
    qk.p[0] = d->query;
    qk.p[1] = d->convolved;
    qk.p[2] = d->key;
    qk.n[0] = d->key_heads;
    qk.n[1] = vh;
    qk.n[2] = d->key_dim;
    qk.n[3] = d->channels;
    rule.p[0] = d->core;
    rule.p[1] = d->query;
    rule.p[2] = d->key;
    rule.p[3] = d->convolved;
    rule.p[4] = d->recurrent;
    rule.p[5] = const_cast<float*>(d->a);
    rule.p[6] = const_cast<float*>(d->b);
    rule.p[7] = const_cast<float*>(d->gates);
    rule.n[0] = d->key_dim;
    rule.n[1] = d->value_dim;
    rule.n[2] = d->key_heads;
    rule.n[3] = vh;
    rule.n[4] = t;
    rule.n[5] = d->channels;
    gate.p[0] = d->gated;
    gate.p[1] = d->core;
    gate.p[2] = const_cast<float*>(d->norm_w);
    gate.p[3] = const_cast<float*>(d->z);
    gate.n[0] = d->value_dim;
    gate.f[0] = d->eps;
    gate.f[1] = 0.f;
    if (int s = qr_run(c, QR_CONV_SILU, d->channels, &conv)) return s;
    if (qr::delta_rule_chunked_ok(rule, vd)) {
        // the chunked rule's prep normalises the convolution's q / k rows
        // itself and stores them to query / key, as DeltaQk would
        ++c->serial;
        auto sc = scope(c, [&] { return std::string("delta_qk+delta_rule_gated chunked"); });
        if (int st = ensure(c, &c->rule_chunks, &c->rule_chunks_len, qr::delta_rule_chunked_scratch(rule),
                            "hipMalloc delta rule chunks"))
            return st;
        if (int st = launched(c, "delta_rule_chunked",
                              qr::run_delta_rule_chunked(c->stream, true, rule, c->rule_chunks, c->rule_chunks_len, true)))
            return st;
    } else {
        if (int s = qr_run(c, QR_DELTA_QK, vh * t, &qk)) return s;
        if (int s = qr_run(c, QR_DELTA_RULE_GATED, vd, &rule)) return s;
    }
    return qr_run(c, QR_RMS_NORM_GATE, vh * t, &gate);
}

// Argmax with fixed partials (no counterpart in the reference's ABI).
int qr_argmax_fixed(Context* c, int rows, const Params* ap) {
    ++c->serial;
    if (!ap) return fail(c, "argmax arguments", -1);
    const Params& a = *ap;
    if (rows < 1 || rows > qr::kArgmaxFixedRows || a.n[0] < 1 || a.n[0] > qr::kArgmaxFixedLength)
        return fail(c, "qr_argmax_fixed: rows must be 1..8 and the row length 1..1048576", -1);
    // (not bracketed by the profiler: its events are created on demand)
    return launched(c, "argmax_fixed", qr::run_argmax_fixed(c->stream, rows, a));
}

// One-launch decode (no counterpart in the reference's ABI).
int qr_decode_plan(Context* c, const QrDecodeDesc* d, QrDecodePlan** out) {
    ++c->serial;
    if (!d || !out) return fail(c, "decode plan arguments", -1);
    const char* why = nullptr;
    int s = qr::decode_plan_create(*d, out, c->stream, &why);
    if (s) {
        std::snprintf(c->error, sizeof(c->error), "%s", why ? why : "one-launch decode unavailable");
        return s;
    }
    if (c->decode_cooperative && (s = qr::decode_plan_cooperative(*out, true))) {
        qr::decode_plan_free(*out);
        *out = nullptr;
        return fail(c, "decode_cooperative: the device has no cooperative launch", s);
    }
    qr::decode_plan_residency(*out, c->decode_residency_test ? 0 : -1, c->decode_residency_auto);
    return 0;
}
// The profile label of a plan's launches.
static std::string step_label(QrDecodePlan* p, const char* what) {
    qr::decode_plan_refresh(p);
    return std::string(what) + (qr::decode_plan_is_cooperative(p) ? " cooperative" : "");
}
int qr_decode_step(Context* c, QrDecodePlan* p, int token, int position) {
    ++c->serial;
    if (!p) return fail(c, "decode step without a plan", -1);
    auto sc = scope(c, [&] { return step_label(p, "decode_step"); });
    if (token < 0) return fail(c, "decode step token", -1);
    return launched(c, "decode step", qr::decode_step(p, token, position, -1, c->stream));
}
int qr_decode_step_capture(Context* c, QrDecodePlan* p, int token, int position, float* capture, int64_t len) {
    ++c->serial;
    if (!p || !capture) return fail(c, "decode step capture without a plan or buffer", -1);
    if (len < int64_t(qr::decode_capture_floats(p))) return fail(c, "decode step capture buffer too short", -1);
    auto sc = scope(c, [&] { return step_label(p, "decode_step_capture"); });
    if (token < 0) return fail(c, "decode step token", -1);
    return launched(c, "decode step", qr::decode_step(p, token, position, -1, c->stream, 0, 0, capture));
}
int qr_decode_rows(Context* c, QrDecodePlan* p, const int32_t* tokens, int n, int position, int first, int snaps) {
    ++c->serial;
    if (!p || !tokens) return fail(c, "decode rows without a plan", -1);
    auto sc = scope(c, [&] { return std::string("decode_rows ") + std::to_string(n); });
    const int st = qr::decode_rows(p, tokens, n, position, first, snaps, c->stream);
    if (st == int(hipErrorNotSupported)) return fail(c, "decode rows: the multi-row kernel does not fit this device", st);
    return launched(c, "decode rows", st);
}
int qr_decode_accept(Context* c, QrDecodePlan* p, int rows) {
    ++c->serial;
    if (!p) return fail(c, "decode accept without a plan", -1);
    auto sc = scope(c, [&] { return std::string("decode_accept"); });
    const int st = qr::decode_accept(p, rows, c->stream);
    if (st == int(hipErrorInvalidValue)) return fail(c, "decode accept: rows beyond the plan's snapshots", st);
    return launched(c, "decode accept", st);
}
int qr_decode_step_row(Context* c, QrDecodePlan* p, int token, int position, int row, int snap) {
    ++c->serial;
    if (!p) return fail(c, "decode step without a plan", -1);
    auto sc = scope(c, [&] { return step_label(p, "decode_step"); });
    if (token < 0 || row < 0 || snap < 0) return fail(c, "decode step token / row / snapshot", -1);
    return launched(c, "decode step", qr::decode_step(p, token, position, -1, c->stream, row, snap));
}
int qr_decode_steps(Context* c, QrDecodePlan* p, int first_token, int position, int n, int32_t* ids, float* bad) {
    ++c->serial;
    if (!p || !ids || !bad || n < 1 || first_token < 0 || position < 0) return fail(c, "decode steps shape", -1);
    int e = qr::decode_history_clear(p, n, c->stream);
    if (e) return launched(c, "decode steps", e);
    for (int k = 0; k < n; ++k) {
        auto sc = scope(c, [&] { return step_label(p, "decode_step"); });
        e = qr::decode_step(p, k == 0 ? first_token : -1, position + k, k, c->stream);
        if (e) return launched(c, "decode steps", e);
    }
    std::vector<float> h(2 * size_t(n));
    e = qr::decode_history_read(p, n, h.data(), c->stream);
    if (e) return launched(c, "decode steps", e);
    float worst = 0.f;
    for (int k = 0; k < n; ++k) {
        const float idx = h[2 * size_t(k)], b = h[2 * size_t(k) + 1];
        const bool ok = b == 0.f && idx >= 0.f && idx < 2147483648.f;  // NaN: the step never wrote its slot
        ids[k] = ok ? int32_t(idx) : -1;
        if (!ok) worst = b == b && b > 0.f ? (b > worst ? b : worst) : 1e30f;
    }
    *bad = worst;
    return 0;
}
void qr_decode_plan_free(Context* c, QrDecodePlan* p) {
    ++c->serial;
    if (c) (void)hipStreamSynchronize(c->stream);
    qr::decode_plan_free(p);
}

int qr_embed_rows(Context* c, float* dst, const float* table, int table_rows, int width, int bf16,
                  const int32_t* ids, int n) {
    ++c->serial;
    if (!dst || !table || !ids || width < 1 || n < 1) return fail(c, "embed_rows shape", -1);
    for (int r = 0; r < n; ++r)
        if (ids[r] < 0 || ids[r] >= table_rows) return fail(c, "embed_rows id out of range", -1);
    auto sc = scope(c, [&] { return std::string(bf16 ? "embed_rows bf16" : "embed_rows f32"); });
    return launched(c, "embed rows", qr::run_embed_rows(c->stream, dst, table, width, bf16 != 0, ids, n));
}

}  // extern "C"
