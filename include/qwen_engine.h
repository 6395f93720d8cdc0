/* C API of the host engine (libqwen_engine.so): a C++ restatement of the
 * reference's Rust device engine, `DeviceModel` / `DeviceRun`
 * (reference src/device.rs:648-2566), driving a qr_* bridge
 * (include/qwen_bridge.h) loaded with dlopen. It issues the same bridge call
 * sequence as `forward_body` (src/device.rs:1740-2378), plus the fp32 arms
 * of `project_all` / `project_norm` / the GLU choice that route fp32 matrices
 * through qr_gemm_f32_group / _add_norm / _glu when the bridge exports them.
 *
 * Every function returning int returns 0 on success and -1 on failure, with
 * the message in qe_last_error(). A failed step, prefill or verify poisons the
 * run until qe_run_reset (src/device.rs:1392-1451).
 */
#ifndef QWEN_ENGINE_H
#define QWEN_ENGINE_H
#include <stddef.h>
#include <stdint.h>

#include "qwen_model.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct QeModel QeModel;
typedef struct QeRun QeRun;
typedef struct QeCheckpoint QeCheckpoint;

/* WeightFormat (src/device.rs:208-219). */
enum QeFormat { QE_F32 = 0, QE_BF16_EXACT = 1, QE_INT8 = 2 };

/* Optional bridge symbols the engine may be told to ignore (as if absent), to
 * exercise the fallbacks of src/device.rs:368-441. */
enum QeDisable {
    QE_NO_F32_FUSIONS = 1,   /* qr_gemm_f32_group / _glu / _add_norm */
    QE_NO_FUSIONS = 2,       /* qr_gemm_bf16_* and qr_gemm_i8_{group,glu,add_norm} */
    QE_NO_DELTA_MIXER = 4,   /* qr_delta_mixer */
    QE_NO_FUSED_OPS = 8,     /* qr_max_op (ops 12-15) */
    QE_NO_ARGMAX = 16,       /* qr_argmax (ops 16-17) */
    QE_NO_SNAPSHOTS = 32,    /* qr_snapshots */
    QE_NO_DECODE_STEP = 64,  /* qr_decode_plan / qr_decode_step */
    QE_NO_EMBED_ROWS = 128,  /* qr_embed_rows */
    QE_NO_PREPARED_GEMM = 256, /* qr_gemm_{f32,bf16,i8}_prepare (prefill projections over planes) */
    QE_NO_PLAIN_DECODE_LAUNCH = 512, /* one-launch decode steps launched cooperatively
                                        (qr_set_option "decode_cooperative"; without it: no plan) */
    QE_NO_DECODE_ROWS = 1024, /* qr_decode_rows (verify rows: one launch per row instead) */
    QE_NO_DECODE_CAPTURE = 2048, /* qr_decode_step_capture (captured steps: the op sequence instead) */
    QE_DECODE_RESIDENCY_TEST = 4096 /* qr_set_option "decode_residency_test": every plain one-launch step
                                       counts as one with a non-resident block, so the plan switches to
                                       cooperative launches after its first step (the switch, tested) */
};

/* Record callback of a captured step: (layer, name, values, n). Names follow
 * `forward_body`'s records ("input_norm", "mixed", "after_mixer", "post_norm",
 * "ffn_product", "ffn", "output"), then "normalized" and "logits". */
typedef void (*qe_record_fn)(void* user, int layer, const char* name, const float* values, int64_t n);

const char* qe_last_error(void);

/* DeviceModel::load_with (src/device.rs:926-934): dlopen `bridge_path`,
 * require qr_abi() == 3 and qr_kind() == expect_kind, upload every tensor
 * (slot order of include/qwen_model.h) in `format`. `disable` is a QeDisable
 * mask. */
QeModel* qe_model_load(const char* bridge_path, int expect_kind, const QwConfig* config,
                       const float* const* tensors, int format, int disable);
/* Releases the model once no run of it is left. The reference's DeviceRun
 * borrows its DeviceModel (src/device.rs:1333-1334), so the model outlives its
 * runs by construction; across a C ABI the free order is the caller's, so runs
 * hold their model and models and runs may be freed in any order. */
void qe_model_free(QeModel* m);
/* qr_info of the bridge context. */
const char* qe_model_info(QeModel* m);
/* weight_summary (src/device.rs:957-965): BF16 matrices, all matrices, device matrix bytes. */
void qe_model_weight_summary(QeModel* m, int64_t* bf16, int64_t* matrices, int64_t* bytes);
/* qr_sync of the bridge context. */
int qe_model_sync(QeModel* m);
/* The bridge's profiler (qr_profile / qr_profile_read), when it has one. */
int qe_model_profile(QeModel* m, int on);
long qe_model_profile_read(QeModel* m, char* out, size_t len);
/* Per-run device budget in bytes (MAX_RUN_BYTES, src/device.rs:855; default 4 GiB). */
void qe_model_set_run_budget(QeModel* m, uint64_t bytes);
/* run_bytes_chunked (src/device.rs:1144-1177). */
uint64_t qe_model_run_bytes(QeModel* m, int64_t capacity, int64_t chunk);

/* new_run_with (src/device.rs:1198-1294). snapshots > 0 is new_run_rollback. */
QeRun* qe_run_new(QeModel* m, int64_t capacity, int64_t chunk, int64_t snapshots);
void qe_run_free(QeRun* r);
int qe_run_reset(QeRun* r);
int64_t qe_run_position(QeRun* r);
/* 1 when uncaptured one-token steps of this run go through the bridge's
 * one-launch decode (qr_decode_plan accepted the run), else 0. */
int qe_run_decode_plan(QeRun* r);

/* DeviceRun::step (src/device.rs:1440-1451); logits: vocab floats. With
 * `record` non-NULL the step is captured (every record read back). */
int qe_step(QeRun* r, uint32_t id, float* logits, qe_record_fn record, void* user);
/* DeviceRun::step_greedy (src/device.rs:1568-1584). */
int qe_step_greedy(QeRun* r, uint32_t id, uint32_t* next);
/* DeviceRun::prefill (src/device.rs:1456-1490); last_logits (vocab floats)
 * is written when ids is non-empty; *has_logits says whether it was. */
int qe_prefill(QeRun* r, const uint32_t* ids, int64_t n, float* last_logits, int* has_logits);
/* verify / verify_rollback (src/device.rs:1495-1531): n rows of logits. */
int qe_verify(QeRun* r, const uint32_t* ids, int64_t n, float* logits);
int qe_verify_rollback(QeRun* r, const uint32_t* ids, int64_t n, float* logits);
/* verify_rollback_greedy (src/device.rs:1595-1610). */
int qe_verify_rollback_greedy(QeRun* r, const uint32_t* ids, int64_t n, uint32_t* picks);
/* accept (src/device.rs:1626-1662). */
int qe_accept(QeRun* r, int64_t rows);
/* unread_logits (src/device.rs:1590-1594): 1 and vocab floats if the last
 * forward was a device-argmax step_greedy, else 0. */
int qe_unread_logits(QeRun* r, float* logits);

/* inspect_state (src/device.rs:2380-2424), one part at a time: which = 0
 * conv history, 1 recurrent state, 2 keys (position * kv * d), 3 values. */
int64_t qe_state_size(QeRun* r, int layer, int which);
int qe_state_read(QeRun* r, int layer, int which, float* out);
/* load_state (src/device.rs:2493-2516) of one part; set_position completes it. */
int qe_state_write(QeRun* r, int layer, int which, const float* values, int64_t n);
int qe_state_set_position(QeRun* r, int64_t position);
/* checkpoint / restore / initial_checkpoint (src/device.rs:2425-2490). */
QeCheckpoint* qe_checkpoint(QeRun* r);
QeCheckpoint* qe_initial_checkpoint(QeRun* r);
int qe_restore(QeRun* r, const QeCheckpoint* c);
void qe_checkpoint_free(QeCheckpoint* c);
int64_t qe_checkpoint_position(const QeCheckpoint* c);

/* Greedy decode loop (decode_greedy_ids, src/generate.rs:135-166) without
 * EOS: feeds `first`, then each pick, n_new tokens in all (n_new - 1
 * forwards), timing the forwards (the reference's decode timing,
 * src/device/cli.rs:797-812). ids: n_new outputs. */
int qe_decode_greedy(QeRun* r, uint32_t first, int64_t n_new, uint32_t* ids, double* seconds);

/* Greedy speculative decoding (generate, src/device/speculative.rs:53-160):
 * prefill `prompt`, then repeatedly draft up to `depth` tokens after the last
 * emitted one, check [last, drafts] in one verify_rollback_greedy pass,
 * emit the leading drafts that equal the model's own picks plus the pick after
 * them, and accept that many rows. Every emitted token is the main model's
 * argmax of a verify row, and verify rows equal decode steps bit for bit, so
 * the output equals plain greedy decoding. Stops after an `eos` token or
 * `max_new` tokens. The run must be fresh (position 0) with at least `depth`
 * snapshots (qe_run_new(..., snapshots >= depth)).
 *
 * A draft source (the reference's `Draft` trait, speculative.rs:162-183,
 * without its hidden-state rows, which feed the MTP head): `absorb` receives
 * the true next tokens (prompt[1..] and the first pick after the prefill, then
 * each pass's emitted tokens); `draft` writes up to k tokens and returns how
 * many (or < 0 on error). */
typedef struct QeDraft {
    void* user;
    int (*absorb)(void* user, const uint32_t* next, int64_t n);
    int64_t (*draft)(void* user, int64_t k, uint32_t* out);
} QeDraft;
/* SpeculativeStats (speculative.rs:30-46): verify passes, drafts offered /
 * accepted at depth j (j < 8), seconds in prefill, drafting and verify. */
typedef struct QeSpecStats {
    int64_t passes;
    int64_t offered[8];
    int64_t accepted[8];
    double prefill_s, draft_s, verify_s;
} QeSpecStats;
int qe_speculative_generate(QeRun* r, const QeDraft* draft, const uint32_t* prompt, int64_t n_prompt,
                            int64_t max_new, int64_t depth, const uint32_t* eos, int64_t n_eos, uint32_t* out,
                            int64_t* n_out, QeSpecStats* stats);
/* A prompt-lookup draft: the longest suffix of the token history (prompt and
 * emitted tokens, up to `max_ngram` tokens) that occurred earlier proposes the
 * tokens that followed its most recent earlier occurrence. No model, so it
 * suits the random-weight configurations; free with qe_draft_ngram_free. */
QeDraft* qe_draft_ngram_new(int64_t max_ngram);
void qe_draft_ngram_free(QeDraft* d);

/* One weight edit (the reference's Edit, src/edit.rs:9-17) on the FFN
 * product of `layer` before its down projection: direction NULL scales
 * product[j] by (1 - coefficient) for every listed column j (unit
 * disabling); a direction d (hidden floats) removes the d component of the
 * down columns w_j, adding -coefficient * d (d . w_j) / (d . d) * product[j]
 * to the FFN output. tensor_name must be
 * "model.language_model.layers.<layer>.mlp.down_proj.weight". */
typedef struct QeEdit {
    int32_t layer;
    const char* tensor_name;
    const int64_t* columns;
    int64_t n_columns;
    const float* direction;
    float coefficient;
} QeEdit;
/* set_edit (src/device.rs:1401-1438): apply `edits` to every following
 * forward of the run (n == 0 removes them; reset keeps them), validated as
 * EditManifest::validate (src/edit.rs:19-58) without the model revision.
 * `tensors` is the host tensor table the model was loaded from (slot order of
 * include/qwen_model.h): the engine copies the down matrices of the edited
 * layers, the fp32 columns the corrections use. Runs with an edit take the
 * op sequence (the product is read back, edited on the host and written
 * back; the capture records gain "ffn_intervened_product"). */
int qe_run_set_edit(QeRun* r, const QeEdit* edits, int64_t n, const float* const* tensors);

/* Checkpoint reader (the reference's read_checkpoint_kept and decode_tensor,
 * src/weights.rs:168-186, 364-466): one streaming pass over a safetensors
 * file, every byte through SHA-256; header checks (contiguous offsets, sizes =
 * shape x dtype size, data ending at the end of the file); F32 decoded, BF16
 * kept as bits, NaN/Inf refused; tensors named in `ignored` hashed and skipped
 * (any dtype). NULL (message in qe_safetensors_error) on any failure, or when
 * expected_sha256 (64 lowercase hex digits) is given and the file does not
 * hash to it. */
typedef struct QeSafetensors QeSafetensors;
enum { QE_ST_F32 = 0, QE_ST_BF16 = 1 };
QeSafetensors* qe_safetensors_read(const char* path, const char* expected_sha256, const char* const* ignored,
                                   int64_t n_ignored);
const char* qe_safetensors_error(void);
void qe_safetensors_free(QeSafetensors* s);
/* The file's SHA-256 (hex). */
const char* qe_safetensors_sha256(const QeSafetensors* s);
/* Tensors in data order: name, dtype (QE_ST_*, -1 for another dtype of an
 * ignored tensor), kept flag, rank and shape (up to 8 dims). */
int64_t qe_safetensors_count(const QeSafetensors* s);
int qe_safetensors_info(const QeSafetensors* s, int64_t i, const char** name, int* dtype, int* kept, int* ndim,
                        int64_t* shape);
/* A kept tensor as n fp32 values (BF16 widened exactly), or a BF16 tensor's bits. */
int qe_safetensors_f32(const QeSafetensors* s, const char* name, float* out, int64_t n);
int qe_safetensors_bf16(const QeSafetensors* s, const char* name, uint16_t* out, int64_t n);

/* Row-wise symmetric int8 quantiser (src/device.rs:220-239) as the engine
 * uploads it. */
void qe_quantize_int8_rows(const float* w, int64_t rows, int64_t cols, float* scales, int8_t* q);

/* Deterministic N(0, std) fill, counter-based: element i of (seed, stream)
 * does not depend on the thread count. */
void qw_synth_normal(float* dst, uint64_t n, uint64_t seed, uint64_t stream, float std_dev, int threads);

#ifdef __cplusplus
}
#endif
#endif
