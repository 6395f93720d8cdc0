// Shared definitions of the gfx950 bridge: wave64 helpers and the launch
// wrappers each kernel translation unit exports to bridge.cpp.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/qwen_bridge.h"

namespace qr {

constexpr int kWave = 64;  // CDNA wavefront

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
// Sum over groups of `width` consecutive lanes (width a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024); every thread gets
// the total. `scratch` holds at least blockDim.x / 64 floats.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < waves; ++w) t += scratch[w];
    return t;
}

// Device math with the reference's branch structure (reference.h:31-40).
__device__ __forceinline__ float sigmoidf_(float x) {
    if (x >= 0.f) return 1.f / (1.f + expf(-x));
    float e = expf(x);
    return e / (1.f + e);
}
__device__ __forceinline__ float siluf_(float x) { return x * sigmoidf_(x); }
__device__ __forceinline__ float softplusf_(float x) { return x > 20.f ? x : log1pf(expf(x)); }

__host__ __device__ inline unsigned ceil_div(long a, long b) { return unsigned((a + b - 1) / b); }

}  // namespace qr

// ---------------------------------------------------------------- launch wrappers
// Each returns 0 or a hipError_t from the launch. `s` is the context stream.
namespace qr {

// gemv.hip -------------------------------------------------------------------
enum class WeightType { F32, BF16, I8 };
struct GemvItem {
    float* y;
    const void* a;  // fp32 / packed bf16 / packed int8 (scales then values)
    int rows;
};
// Y_i[batch, rows_i] = X[batch, cols] . A_i^T for up to kGroupMax items.
constexpr int kGroupMax = 8;
int gemv_group(hipStream_t s, WeightType t, const GemvItem* items, int n, const float* x, int cols, int batch);
// product[batch, rows] = silu(X G^T) * (X U^T)
int gemv_glu(hipStream_t s, WeightType t, float* product, const void* gate, const void* up, const float* x, int rows,
             int cols, int batch);
// One token: y = A x, then sum = u + v and norm = RmsNorm(sum) (weight, eps, offset) by the last block.
int gemv_add_norm(hipStream_t s, WeightType t, float* y, const void* a, const float* x, int rows, int cols,
                  const QrAddNormPost& post, unsigned* ticket);

// gemm.hip -------------------------------------------------------------------
// Y[batch, rows] = X[batch, cols] . A^T (prefill). `work`: bridge scratch of
// at least gemm_scratch(...) floats (K-split partials).
int gemm(hipStream_t s, WeightType t, float* y, const void* a, const float* x, int rows, int cols, int batch,
         float* work, size_t work_len);
size_t gemm_scratch(WeightType t, int rows, int cols, int batch);
bool gemm_preferred(WeightType t, int rows, int cols, int batch);
// gemm_p3.hip -----------------------------------------------------------------
// P3 planes: the three BF16 split planes (x = x0 + x1 + x2) of a [rows, cols]
// fp32 matrix in MFMA fragment order, rows padded to a multiple of 256 (pad
// rows zero): the 32 x 16 fragment (rows 32 rt.., k 16 kt..) of plane p is
// 512 contiguous BF16 at ((rt cols/16 + kt) 3 + p) 512, element (row, k) at
// lane (row % 32) + 32 ((k / 8) % 2), position k % 8.
__host__ __device__ inline int p3_rows(int rows) { return (rows + 255) / 256 * 256; }
__host__ __device__ inline bool p3_cols_ok(int cols) { return cols >= 32 && cols % 32 == 0; }
__host__ __device__ inline size_t p3_index(int row, int k, int plane, int kt) {
    return ((size_t(row >> 5) * size_t(kt) + size_t(k >> 4)) * 3 + size_t(plane)) * 512 +
           size_t((row & 31) + 32 * ((k >> 3) & 1)) * 8 + size_t(k & 7);
}
size_t p3_elements(int rows, int cols);
// fp32 [rows, cols] -> P3 planes (cols % 32 == 0, 16-byte aligned pointers).
int p3_split(hipStream_t s, __bf16* out, const float* in, int rows, int cols);
// A matrix exact in BF16 as ONE plane in the same fragment order ("P1":
// element (row, k) at p3_index(row, k, 0, kt) with one plane per fragment
// slot, i.e. ((row / 32) kt + k / 16) 512 + ...), from the packed BF16 words
// of the reference's upload_bf16; p1_elements(rows, cols) BF16.
size_t p1_elements(int rows, int cols);
int p1_from_bf16(hipStream_t s, __bf16* out, const void* packed, int rows, int cols);
// The same plane from the int8 values of a [rows fp32 scales | int8 values]
// matrix (the reference's upload_int8); the scales are applied after the sum.
int p1_from_i8(hipStream_t s, __bf16* out, const void* packed, int rows, int cols);
// Y[M, N] = X W^T from the P3 planes of X (M rows) and W's planes (N rows; 3,
// or wplanes = 1 for P1), K % 32 == 0, each column times scale[n] after the
// sum when `scale` is set (int8 weights, P1 only); `work` holds at least
// p3_gemm_scratch(M, N, K, wplanes) floats (K-chunk partials).
int p3_gemm(hipStream_t s, float* y, const __bf16* xp, const __bf16* wp, int M, int N, int K, float* work,
            size_t work_len, int wplanes = 3, const float* scale = nullptr);
size_t p3_gemm_scratch(int M, int N, int K, int wplanes = 3);
// The combined planes of a GLU (2 rows x cols; rows % 128 == 0) from the
// planes (3, or 1 for P1) of gate and up: 64 gate rows, then the same 64 up
// rows, and so on.
int p3_glu_interleave(hipStream_t s, __bf16* out, const __bf16* gate, const __bf16* up, int rows, int cols,
                      int planes = 3);
// product[M, rows] = silu(X G^T) * (X U^T) from X's P3 planes and the combined
// planes; when `planes` is set, the product's P3 planes too (rows / 16 k
// tiles). `work`: at least p3_glu_scratch(M, rows, K, wplanes) floats.
int p3_gemm_glu(hipStream_t s, float* product, __bf16* planes, const __bf16* xp, const __bf16* wglu, int M, int rows,
                int K, float* work, size_t work_len, int wplanes = 3, const float* scale_gate = nullptr,
                const float* scale_up = nullptr);
size_t p3_glu_scratch(int M, int rows, int K, int wplanes = 3);

// Y1 = X A1^T and (rows2 > 0) Y2 = X A2^T in one launch for fp32 (or packed
// BF16 / int8, cols % 16 == 0) matrices of at most 16 rows and 1024 columns
// (the DeltaNet a / b projections of prefill), when gemm_ab_ok holds for each.
bool gemm_ab_ok(WeightType t, const void* a, const float* x, int rows, int cols, int batch);
int gemm_ab(hipStream_t s, float* y1, const float* a1, int rows1, float* y2, const float* a2, int rows2,
            const float* x, int cols, int batch, WeightType t = WeightType::F32);
// product[batch, rows] = silu(X G^T) * (X U^T) in one kernel (prefill, any weight format).
bool gemm_glu_fused(WeightType t, const void* gate, const void* up, const float* x, int rows, int cols, int batch);
int gemm_glu(hipStream_t s, WeightType t, float* product, const void* gate, const void* up, const float* x, int rows,
             int cols, int batch);

// ops.hip --------------------------------------------------------------------
int run_elementwise(hipStream_t s, int op, int count, const Params& a);
int run_rms_family(hipStream_t s, int op, int groups, const Params& a);
// RmsNorm / AddRmsNorm / RmsNormGate whose output is also written as the P3
// planes of rows of `width` values (a multiple of the group size and of 32
// that divides the output: groups * d / width rows); hipErrorNotSupported
// (nothing launched) when the op, width or alignment has no such form.
int run_rms_family_planes(hipStream_t s, int op, int groups, const Params& a, __bf16* planes, int width);
int run_conv_silu(hipStream_t s, int count, const Params& a);
int run_delta_qk(hipStream_t s, int count, const Params& a);
int run_delta_rule(hipStream_t s, bool gated, int count, const Params& a);
// `denom`: device table of theta^(2i / rot), i < rot / 2 (see rope_lds).
int run_attention_qkv(hipStream_t s, int op, int count, const Params& a, const float* denom);
int run_embed(hipStream_t s, int op, int count, const Params& a);
// dst[r] = table row ids[r] (fp32, or packed BF16 widened), r < n; ids on the host.
int run_embed_rows(hipStream_t s, float* dst, const void* table, int width, bool bf16, const int32_t* ids, int n);
int run_argmax(hipStream_t s, int rows, const Params& a, float* parts, size_t parts_len);
// The same argmax with its partials in a fixed per-device array: at most
// kArgmaxFixedRows rows of kArgmaxFixedLength entries; allocates nothing.
// argmax_fixed_init resolves the array's device address for the current
// device (once per device).
constexpr int kArgmaxFixedRows = 8, kArgmaxFixedLength = 1 << 20;
int argmax_fixed_init();
int run_argmax_fixed(hipStream_t s, int rows, const Params& a);
size_t argmax_parts_needed(int rows, int n);

// attention.hip --------------------------------------------------------------
// AttentionRead (op 10). `scratch` is the bridge's own partials buffer.
int run_attention_read(hipStream_t s, int heads_count, const Params& a, float* scratch, size_t scratch_len);
size_t attention_scratch_needed(const Params& a);

// decode.hip -----------------------------------------------------------------
// One-launch decode step (qr_decode_plan / qr_decode_step).
const char* decode_unsupported(const QrDecodeDesc& d);
int decode_plan_create(const QrDecodeDesc& d, QrDecodePlan** out, hipStream_t s, const char** why);
void decode_plan_free(QrDecodePlan* p);
// Launch the plan's steps cooperatively (on) or as plain launches (off, the
// default); hipErrorNotSupported when the device has no cooperative launch.
int decode_plan_cooperative(QrDecodePlan* p, bool on);
// The residency check of plain launches: a launch whose blocks start `ticks`
// (100 MHz; < 0: unchanged, default 5000) or more apart sets the plan's
// flag, and with `automatic` (default) the plan launches cooperatively from
// its next step on.
void decode_plan_residency(QrDecodePlan* p, int ticks, bool automatic);
// True when the plan's steps launch cooperatively (chosen, or switched to by
// the residency check).
bool decode_plan_is_cooperative(const QrDecodePlan* p);
// Applies a set residency flag (the switch to cooperative launches); every
// launch does this first.
void decode_plan_refresh(QrDecodePlan* p);
// token -1: the previous launch's argmax (read on the device). slot >= 0: the
// step's [argmax, non-finite count] also goes to history slot `slot`.
// slot >= 0: the chained-steps history slot; row: logits / picks row; snap: snapshot copy (0: none).
// cap: when set, the step's per-layer records (decode_capture_floats(layers) floats).
int decode_step(QrDecodePlan* p, int token, int position, int slot, hipStream_t s, int row = 0, int snap = 0,
                float* cap = nullptr);
size_t decode_capture_floats(const QrDecodePlan* p);
// Up to 4 consecutive tokens in one launch (qr_decode_rows).
int decode_rows(QrDecodePlan* p, const int* tokens, int n, int position, int first, int snaps, hipStream_t s);
int decode_history_clear(QrDecodePlan* p, int n, hipStream_t s);
// accept for every DeltaNet layer of the plan in one launch: snapshot copy
// `rows` (1..snapshots) of each recurrent state and conv history becomes copy 0.
int decode_accept(QrDecodePlan* p, int rows, hipStream_t s);
int decode_history_read(QrDecodePlan* p, int n, float* out, hipStream_t s);

// delta_chunk.hip ------------------------------------------------------------
// DeltaRule / DeltaRuleGated over a prefill chunk in the WY form (key_dim ==
// value_dim == 128, no snapshots, at least kChunkMinTokens tokens).
constexpr int kChunkMinTokens = 16;
bool delta_rule_chunked_ok(const Params& a, int count);
size_t delta_rule_chunked_scratch(const Params& a);  // floats
// qkn: q and k taken from the convolution output (slot 3) and normalised as
// DeltaQk does, the normalised rows also stored to slots 1 and 2.
int run_delta_rule_chunked(hipStream_t s, bool gated, const Params& a, float* scratch, size_t len, bool qkn = false);

// deltanet.hip ---------------------------------------------------------------
// qr_delta_mixer for one token (decode) when the shape allows; returns -1 if not handled.
int delta_mixer_decode(hipStream_t s, const QrDelta& d);
bool delta_mixer_decode_ok(const QrDelta& d);

}  // namespace qr
