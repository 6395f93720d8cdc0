/* The device bridge C ABI (version 3) that the reference's Rust device engine
 * loads with dlopen (reference src/device.rs:322-474), exported here by the
 * MI355X (gfx950) bridge libqwen_mi355x.so. Every entry point below replaces
 * the one the reference's ROCm bridge exports (native/rocm/bridge.cpp); the
 * comment of each cites the reference declaration it stands in for and the
 * engine call site that binds it.
 *
 * Conventions (reference src/device.rs:33-190, native/rocm/bridge.cpp:354-910):
 *   - every length is in 32-bit words (BF16 matrices pack two values per word,
 *     element 2i in the low half; int8 matrices are `rows` fp32 scales followed
 *     by the row-major int8 values, four per word, the last word zero-padded);
 *   - every call returns 0 on success; otherwise qr_error() holds the message;
 *   - all work of one context is ordered on one HIP stream; qr_read/qr_sync
 *     synchronise it and are where asynchronous faults surface;
 *   - one host thread per context.
 */
#ifndef QWEN_BRIDGE_H
#define QWEN_BRIDGE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct Context Context;

/* Op arguments (reference native/rocm/reference.h:29, src/device.rs:33-38). */
typedef struct Params {
    float* p[8];
    int32_t n[8];
    float f[4];
} Params;

/* qr_run op codes (reference native/rocm/reference.h:21-24, src/device.rs:39-73). */
enum QrOp {
    QR_RMS_NORM = 1, QR_ADD = 2, QR_SILU_PRODUCT = 3, QR_CONV_SILU = 4, QR_DELTA_QK = 5, QR_DELTA_GATES = 6,
    QR_DELTA_RULE = 7, QR_ATTENTION_QUERY = 8, QR_ATTENTION_KV = 9, QR_ATTENTION_READ = 10, QR_EMBED_BF16 = 11,
    QR_ADD_RMS_NORM = 12, QR_RMS_NORM_GATE = 13, QR_DELTA_RULE_GATED = 14, QR_ATTENTION_QUERY_KV = 15,
    QR_ARGMAX = 16, QR_EMBED_BF16_PICKED = 17
};

/* Bridge kinds returned by qr_kind (reference src/device.rs:74-80). */
enum QrKind { QR_KIND_CPU_TEST = 0, QR_KIND_ROCM = 1, QR_KIND_METAL = 2, QR_KIND_CUDA = 3 };

/* One entry of a grouped projection (reference src/device.rs:116-122). */
typedef struct QrProjection {
    float* y;
    const float* a;
    int32_t rows;
} QrProjection;

/* qr_delta_mixer arguments (reference src/device.rs:125-151, bridge.cpp:735-742). */
typedef struct QrDelta {
    float* convolved; const float* projected; const float* conv_w; float* conv_state;
    float* query; float* key; float* core; float* recurrent;
    const float* a; const float* b; const float* gates;
    float* gated; const float* norm_w; const float* z;
    int32_t key_heads, value_heads, key_dim, value_dim, kernel, tokens, channels;
    float eps;
} QrDelta;

/* Add + RmsNorm after a one-token GEMV (reference src/device.rs:153-163, bridge.cpp:801). */
typedef struct QrAddNormPost {
    float* sum; const float* u; const float* v; const float* weight; float* norm;
    float eps; float offset;
} QrAddNormPost;

/* ---- mandatory symbols (reference src/device.rs:341-367,442-450) ---- */

/* ABI version, 3 (bridge.cpp:355). */
int qr_abi(void);
/* 1 = ROCm (bridge.cpp:364-372); the engine refuses any other kind in production. */
int qr_kind(void);
/* Context with its own stream on device 0 (bridge.cpp:375-411). */
int qr_create(Context** out);
/* n_floats zero-filled device words (bridge.cpp:457-466). */
int qr_alloc(Context* c, float** p, size_t n_floats);
/* bridge.cpp:478-486 */
void qr_free(Context* c, float* p);
/* Host -> device, synchronous: the host slice may die on return (bridge.cpp:487-497). */
int qr_write(Context* c, float* dst, const float* host, size_t n);
/* Device -> host, synchronises the stream (bridge.cpp:498-517). */
int qr_read(Context* c, float* host, const float* src, size_t n);
/* Device -> device, asynchronous on the stream (bridge.cpp:518-528). */
int qr_copy(Context* c, float* dst, const float* src, size_t n);
/* Runs op `op` over `count` items (bridge.cpp:529-570; slot semantics reference.h:117-232). */
int qr_run(Context* c, int op, int count, const Params* a);
/* y[rows] = A[rows, cols] x, fp32 A (bridge.cpp:571-583). */
int qr_gemv(Context* c, float* y, const float* a, const float* x, int rows, int cols);
/* As qr_gemv with BF16 A (bridge.cpp:654-656). */
int qr_gemv_bf16(Context* c, float* y, const float* packed, const float* x, int rows, int cols);
/* Y[batch, rows] = X[batch, cols] A^T, fp32 A (bridge.cpp:584-602). */
int qr_gemm(Context* c, float* y, const float* a, const float* x, int rows, int cols, int batch);
/* As qr_gemm with BF16 A (bridge.cpp:603-619). */
int qr_gemm_bf16(Context* c, float* y, const float* packed, const float* x, int rows, int cols, int batch);
/* bridge.cpp:427-435 */
int qr_sync(Context* c);
/* NUL-terminated, owned by the context (bridge.cpp:373). */
const char* qr_error(Context* c);
/* Device and runtime description (bridge.cpp:374,405-407). */
const char* qr_info(Context* c);
/* bridge.cpp:436-456 */
void qr_destroy(Context* c);

/* ---- optional symbols (reference src/device.rs:368-441) ---- */

/* Highest qr_run op run by qr_run, 15 (bridge.cpp:356-358). */
int qr_max_op(void);
/* 1: ConvSilu n3 / DeltaRule(Gated) n6 store per-token state snapshots (bridge.cpp:359-361). */
int qr_snapshots(void);
/* 2: ops Argmax and EmbedBf16Picked (bridge.cpp:362-363). */
int qr_argmax(void);
/* Engine options; "attention_f16" is refused (RDNA3 WMMA only) (bridge.cpp:412-426).
 * "decode_cooperative" (0/1, this bridge's own): one-launch decode plans made after the
 * call launch their steps cooperatively (the runtime guarantees the 256 blocks are
 * resident together, about 20 us more per step) instead of as plain launches, which
 * need a device no other stream or process is using at that moment. */
int qr_set_option(Context* c, const char* name, int value);
/* int8 per-row weights: Y[batch, rows] = scale[r] * (X Q^T) (bridge.cpp:620-653). */
int qr_gemm_i8(Context* c, float* y, const float* packed, const float* x, int rows, int cols, int batch);
/* n projections of one X (bridge.cpp:657-700 for BF16, 838-866 for int8). */
int qr_gemm_bf16_group(Context* c, int n, const QrProjection* items, const float* x, int cols, int batch);
int qr_gemm_i8_group(Context* c, int n, const QrProjection* items, const float* x, int cols, int batch);
/* product = silu(X G^T) * (X U^T); gate_y/up_y are scratch (bridge.cpp:701-729, 867-885). */
int qr_gemm_bf16_glu(Context* c, float* product, float* gate_y, float* up_y, const float* gate, const float* up,
                     const float* x, int rows, int cols, int batch);
int qr_gemm_i8_glu(Context* c, float* product, float* gate_y, float* up_y, const float* gate, const float* up,
                   const float* x, int rows, int cols, int batch);
/* One-token GEMV, then post->sum = u + v and post->norm = RmsNorm(sum) (bridge.cpp:797-827, 886-909). */
int qr_gemm_bf16_add_norm(Context* c, float* y, const float* packed, const float* x, int rows, int cols,
                          const QrAddNormPost* post);
int qr_gemm_i8_add_norm(Context* c, float* y, const float* packed, const float* x, int rows, int cols,
                        const QrAddNormPost* post);
/* ConvSilu, DeltaQk, DeltaRuleGated and RmsNormGate of one DeltaNet layer (bridge.cpp:730-796). */
int qr_delta_mixer(Context* c, const QrDelta* d);

/* fp32 versions of the grouped / GLU / add-norm projections, with the int8
 * signatures. The reference's engine picks the fused calls only for BF16 and
 * int8 matrices (src/device.rs:779-786, 1801-1808, 2153-2160); these let an
 * fp32-weight run take the same fused route through a three-site `m.f32` arm
 * in `project_all`, `project_norm` and the GLU choice. Each output equals the
 * separate qr_gemm / qr_gemv calls (and op SiluProduct / AddRmsNorm) it
 * replaces, up to fp32 summation order. */
int qr_gemm_f32_group(Context* c, int n, const QrProjection* items, const float* x, int cols, int batch);
int qr_gemm_f32_glu(Context* c, float* product, float* gate_y, float* up_y, const float* gate, const float* up,
                    const float* x, int rows, int cols, int batch);
int qr_gemm_f32_add_norm(Context* c, float* y, const float* a, const float* x, int rows, int cols,
                         const QrAddNormPost* post);

/* Prepared fp32 matrices (no counterpart in the reference's ABI; optional:
 * an engine may call qr_gemm_f32_prepare once after uploading an fp32 matrix
 * `a` of rows x cols, 16-byte aligned). When cols % 32 == 0 the bridge keeps
 * the matrix's three-way BF16 split planes in MFMA fragment order (6 bytes per
 * element) and runs every qr_gemm / qr_gemm_f32_group / qr_gemm_f32_glu
 * projection of `a` over at least 64 tokens on its own BF16-MFMA kernel over
 * them (gemm_p3.hip: the six part products of the split, fp32 accumulation and
 * output, hence fp32 accuracy; a GLU of two prepared matrices with rows % 128
 * == 0 runs gate, up and the silu product as one kernel, gate_y and up_y
 * untouched). Other column counts prepare nothing (returns 0). The planes are
 * dropped by qr_gemm_f32_release(a), by qr_free(a), and by any qr_write /
 * qr_copy into the matrix's range; unprepared matrices take the split-BF16
 * kernel. */
int qr_gemm_f32_prepare(Context* c, const float* a, int rows, int cols);
int qr_gemm_f32_release(Context* c, const float* a);
/* Prepared BF16 matrices (no counterpart in the reference's ABI; optional,
 * as qr_gemm_f32_prepare): `packed` is a rows x cols matrix in the words of
 * the reference's upload_bf16 (src/device.rs:535-549; element 2i in the low
 * half of word i), 16-byte aligned. When cols % 32 == 0 the bridge keeps its
 * one plane in the same fragment order (2 bytes per element) and runs every
 * qr_gemm_bf16 / qr_gemm_bf16_group / qr_gemm_bf16_glu projection of it over
 * at least 64 tokens on the same kernels with three part products (x's three
 * planes times the exact BF16 weight). Released and invalidated as prepared
 * fp32 matrices (qr_gemm_f32_release takes either). */
int qr_gemm_bf16_prepare(Context* c, const float* packed, int rows, int cols);
/* Prepared int8 matrices (no counterpart in the reference's ABI; optional, as
 * qr_gemm_bf16_prepare): `packed` is the reference's upload_int8 layout
 * (src/device.rs:550-561: rows fp32 scales, then the int8 values four per
 * word). The bridge keeps the values' one plane (integers are exact in BF16);
 * qr_gemm_i8 / qr_gemm_i8_group / qr_gemm_i8_glu over at least 64 tokens run
 * the plane kernels and scale each output by its row's scale after the sum
 * (scale * sum(q x), as qr_gemm_i8). Released and invalidated as above. */
int qr_gemm_i8_prepare(Context* c, const float* packed, int rows, int cols);

/* One decode token in one launch (no counterpart in the reference's ABI; the
 * engine calls it from `forward` when t == 1, nothing is captured, the
 * matrices are all fp32 or all int8 and the bridge accepted the plan, instead
 * of the op sequence of src/device.rs:1740-2378, which it computes identically
 * up to fp32 summation order). The plan registers every weight, state and output
 * buffer of one run once; each step embeds `token`, runs all layers at
 * `position` (appending K/V there and advancing the DeltaNet states), writes
 * the vocabulary logits to `logits` and [argmax index, non-finite count] to
 * `picks` (op Argmax's output, reference.h:222-230). */
typedef struct QrDecodeLayer {
    int32_t attention;  /* 1 full attention, 0 Gated DeltaNet */
    const float* input_norm; const float* post_norm;
    const float* gate; const float* up; const float* down;
    /* attention */
    const float* q; const float* k; const float* v; const float* o;
    const float* qk_norm;            /* [q_norm | k_norm] */
    float* keys; float* values;      /* caches [capacity, kv_heads, head_dim] */
    /* Gated DeltaNet */
    const float* qkv; const float* z; const float* a; const float* b;
    const float* conv_w; const float* gates; /* [dt | A_log] */ const float* norm_w; const float* out;
    float* conv_state; float* recurrent;
} QrDecodeLayer;
typedef struct QrDecodeDesc {
    int32_t hidden, intermediate, vocab, layers, heads, kv_heads, head_dim, rotary_dim;
    int32_t key_heads, value_heads, key_dim, value_dim, conv_kernel, capacity;
    float eps, theta;
    const float* embedding;  /* [vocab, hidden]: the lookup rows */
    const float* lm_head;    /* vocabulary projection, [vocab, hidden] */
    const float* final_norm;
    float* logits;           /* [vocab] */
    float* picks;            /* [2] */
    const QrDecodeLayer* layer;
    /* Matrix format of every layer matrix and of lm_head: QR_DECODE_F32,
     * QR_DECODE_BF16 (the reference's upload_bf16_bits packing,
     * src/device.rs:535-549: two to a word, element 2i in the low half; a
     * tied LM head is the BF16 embedding table) or QR_DECODE_INT8 (the
     * reference's upload_int8 packing, src/device.rs:550-561: rows fp32
     * scales, then the int8 values row-major, four to a word). */
    int32_t weights;
    int32_t embedding_bf16;  /* embedding is packed BF16 (element 2i in the low half of word i) */
    /* Rows of `logits` ([rows, vocab]) and `picks` ([rows, 2]) a launch may
     * write (1..8), and the snapshot copies that follow each DeltaNet layer's
     * conv_state and recurrent state (0..7; copy s of a [n] state at
     * state + s * n, the layout of the ops' snapshot mode). */
    int32_t rows, snapshots;
} QrDecodeDesc;
enum { QR_DECODE_F32 = 0, QR_DECODE_BF16 = 1, QR_DECODE_INT8 = 2 };
typedef struct QrDecodePlan QrDecodePlan;
/* Non-zero (with qr_error set) when this bridge has no one-launch decode for the shape. */
int qr_decode_plan(Context* c, const QrDecodeDesc* d, QrDecodePlan** out);
int qr_decode_step(Context* c, QrDecodePlan* p, int token, int position);
/* n greedy one-launch steps queued back to back: step k runs at position + k
 * on first_token (k = 0) or on step k-1's argmax, which the kernel reads from
 * the device, so the host does not wait between steps. ids[k] = step k's
 * argmax (-1 where the step failed); *bad = 0 when every step's logits were
 * finite, else the largest non-finite count (1e30 when a step did not finish).
 * No counterpart in the reference's ABI: its step_greedy reads each argmax
 * back before the next step (src/device.rs:1568-1584); the tokens are the
 * same. */
int qr_decode_steps(Context* c, QrDecodePlan* p, int first_token, int position, int n, int32_t* ids, float* bad);
/* One launch of the step for a verify row: token at position, its logits in
 * logits row `row` and [argmax, non-finite count] in picks row `row`, and when
 * snap > 0 the DeltaNet states after this token also written to snapshot copy
 * `snap`. Every row is the same kernel as qr_decode_step, so a verify row is
 * bit for bit the decode step of its position (the reference's contract for
 * verify rows, native/rocm/bridge.cpp:197-215, src/device.rs:1514-1531). No
 * counterpart in the reference's ABI. */
int qr_decode_step_row(Context* c, QrDecodePlan* p, int token, int position, int row, int snap);
/* qr_decode_step with the per-layer records of a captured forward also
 * written to `capture` (device memory of len floats, at least layers *
 * (6 hidden + intermediate) + hidden): layer L's records at capture +
 * L (6 hidden + intermediate), in the order of src/device.rs:1748-1761's
 * records (input_norm, mixed, after_mixer, post_norm [hidden each],
 * ffn_product [intermediate], ffn, output [hidden each]), then the final norm
 * [hidden]. The engine reads them back and reports them as the op sequence's
 * capture would (the same values up to fp32 summation order), so a captured
 * step keeps the one-launch kernel. No counterpart in the reference's ABI,
 * which captures on the op sequence. */
int qr_decode_step_capture(Context* c, QrDecodePlan* p, int token, int position, float* capture, int64_t len);
/* Part of a verify pass, n = 1..4 consecutive tokens in ONE launch, the
 * weights read once for all rows: row r is tokens[r] at position + r (logits
 * row first + r, [argmax, non-finite count] in picks row first + r), and when
 * first + r < snaps its DeltaNet states also go to snapshot copy first + r + 1.
 * Every row is computed with the per-lane arithmetic of qr_decode_step at its
 * position (the delta rule walks the rows in order, row r's attention is split
 * as a one-row step at position + r would be and sees the new keys / values
 * of rows <= r), so a row is bit for bit the decode step of its position, as
 * the reference's fixed-count verify GEMV keeps each row's order
 * (native/rocm/kernels.h:124-170, native/rocm/bridge.cpp:197-215).
 * first + n <= the plan's rows, snaps <= its snapshots. No counterpart in the
 * reference's ABI. */
int qr_decode_rows(Context* c, QrDecodePlan* p, const int32_t* tokens, int n, int position, int first, int snaps);
/* accept (src/device.rs:1626-1662) of a verify pass in one launch: for every
 * DeltaNet layer of the plan, snapshot copy `rows` (1..snapshots) of the
 * recurrent state and of the conv history replaces copy 0, as the engine's
 * two qr_copy calls per layer would (36 calls at the 0.8B shape). No
 * counterpart in the reference's ABI. */
int qr_decode_accept(Context* c, QrDecodePlan* p, int rows);
void qr_decode_plan_free(Context* c, QrDecodePlan* p);

/* Op 16 (Argmax) without any allocation: the same slot meanings and result
 * as qr_run(c, QR_ARGMAX, rows, a) (p[0]: [rows, 2] out, p[1]: [rows, n[0]]
 * logits), but the per-slice partials live in a fixed per-device array of the
 * library (12 KiB, held until the process ends), so no call allocates device
 * memory. At most 8 rows of at most 1,048,576 entries (larger inputs are
 * refused with an error). Calls that overlap on one device share the array
 * and race. No counterpart in the reference; for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops). */
int qr_argmax_fixed(Context* c, int rows, const Params* a);

/* Embedding rows of a prefill chunk in one call: dst[r, 0..width) = row
 * ids[r] of `table` for r < n (ids on the host, each checked against
 * table_rows; bf16 != 0: `table` is packed BF16 and the rows are widened).
 * Replaces the per-token qr_copy (fp32) or EmbedBf16 op (BF16) of the
 * reference's DeviceRun::forward (src/device.rs:1716-1732) with the same
 * result; no counterpart in the reference's ABI. */
int qr_embed_rows(Context* c, float* dst, const float* table, int table_rows, int width, int bf16,
                  const int32_t* ids, int n);

/* In-bridge profiler: while on, every bridge call is bracketed by a hipEvent
 * pair on the context stream and the durations are summed per call label
 * (kernel family and shape). No counterpart in the reference's ABI: its
 * bridge has the same profiler behind QWEN_ROCM_PROFILE
 * (native/rocm/bridge.cpp:55-139), which this bridge also honours (table on
 * stderr at qr_destroy). For benchmarks that time kernels on the stream the
 * kernels run on. */
int qr_profile(Context* c, int on);
/* Totals since qr_profile(c, 1), one line per label: "calls\ttotal_ms\tlabel\n".
 * Returns the buffer size the whole text needs (truncated to len), -1 on error. */
long qr_profile_read(Context* c, char* out, size_t len);

#ifdef __cplusplus
}
#endif
#endif
