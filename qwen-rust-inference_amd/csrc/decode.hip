// One decode token of the Qwen3.5-0.8B hybrid in ONE launch on gfx950
// (qr_decode_plan / qr_decode_step). It computes what the bridge's op
// sequence for one token computes (the engine's forward_body; arithmetic of
// every step as in native/rocm/reference.h), with fp32 sums in its own order.
//
// Why one launch: at batch 1 the step is a chain of ~130 dependent stages
// (each projection needs the whole previous vector). As separate kernels each
// stage pays a dispatch, a ramp-up and a drain (~2-5 us for the small
// matrices) and the step cannot approach the HBM roofline. Here 256 blocks of
// 8 waves stay resident and walk the stage list together. The kernel needs
// all 256 blocks resident at once (one per CU: 256 VGPRs per lane leave room
// for one 8-wave block per CU). A plain launch gets that on a device no other
// stream or process is using (the previous step on the same stream has
// finished, so every CU is free when the grid is dispatched); a cooperative
// launch has the runtime guarantee it, at about 20 us more per step, and is
// chosen per plan (decode_plan_cooperative). Either way a block that is not
// resident makes the others' polls time out: the step then fails (below)
// instead of hanging.
//
// Structure:
//   * The phase list: per DeltaNet layer in-proj + conv, mixer (+ z rows),
//     out-proj, GLU, down; per attention layer QKV, attention, combine,
//     o-proj, GLU, down; then lm_head and argmax. All 2048 waves take part in
//     every phase; a phase's rows are spread wave-major over the blocks
//     (unit u = wave * 256 + block), so partial phases still use every CU.
//   * A wave's share of any phase's weights (and DeltaNet state / KV rows,
//     none of which depend on this token's activations) is at most 16 x 16
//     bytes per lane. Right after a wave finishes phase p it issues the loads
//     of phase p + 1 into that register buffer, so HBM streams the next stage
//     while the wave waits for that stage's inputs.
//   * There is no grid barrier. Every activation crossing blocks is stored as
//     a (value, tag) pair in ONE 8-byte system-coherent write (sc0 sc1,
//     write-through), tag = (launch epoch, producing phase). A consumer polls
//     the pairs it needs until every tag is the expected one: data and
//     readiness arrive in the same read. Each buffer is rewritten only after
//     every reader of its previous contents has produced something the writer
//     transitively needs, so a consumer never sees a later phase's value.
//     (The attention split partials are plain stores published by a tagged
//     (max, sum) pair written after an s_waitcnt.)
//   * Broadcast vectors are staged once per block in LDS (double-buffered by
//     phase parity; the barriers of each phase keep the block's waves within a
//     phase of each other, so a buffer is never rewritten while read). A
//     vector stays readable until the block stages into its buffer again, so
//     later phases take the residual (and MIX its input) from there instead of
//     polling it.
//   * Every poll is bounded by the 100 MHz real-time counter; on a time-out a
//     lane records an error (picks[1] = 1e30, a non-finite count the engine
//     refuses), the block's waves leave together after their next s_barrier,
//     and blocks waiting on them time out in turn.
#include <cstddef>
#include <cstring>
#include <mutex>
#include <utility>
#include <vector>

#include "common.h"

namespace qr {
namespace dec {

// Geometry this kernel is written for (Qwen3.5-0.8B text model).
constexpr int H = 1024, I = 3584, HD = 256, NH = 8, NKV = 2, ROT = 64;
constexpr int DK = 128, DV = 128, VH = 16, KH = 16, CONVK = 4;
constexpr int KD = KH * DK;         // 2048
constexpr int VD = VH * DV;         // 2048
constexpr int CH = 2 * KD + VD;     // 6144 conv channels
constexpr int QROWS = 2 * NH * HD;  // 4096 rows of q_proj ([Q | gate] per head)
constexpr int KVR = NKV * HD;       // 512
constexpr int DIN_ROWS = CH + 2 * VH;       // 6176 rows of qkv | a | b (z: in the mixer phase)
constexpr int AQKV_ROWS = QROWS + 2 * KVR;  // 5120
constexpr int BLOCKS = 256, WAVES = 8, THREADS = 64 * WAVES;
constexpr int NW = BLOCKS * WAVES;  // 2048 waves
constexpr int WBUF = 16;            // prefetch buffer, 16-byte entries per lane
constexpr int SPAN = 8;             // attention positions per K/V chunk (2 steps of 4)
constexpr int KVE = 2 * SPAN;       // 16-byte entries per lane of one K/V chunk
constexpr int SMAX = 256;           // attention splits per KV head
constexpr int QPG = NH / NKV;       // query heads per KV head: the waves of one attention slot
constexpr int MAXPH = 6 * 64 + 2;
// Rows of a multi-row step (decode_rows_kernel: a verify pass of up to NRMAX
// consecutive tokens with the weights read once).
constexpr int NRMAX = 4;
// Matrix formats (the W template parameter): fp32; BF16 packed two to a word
// (element 2i in the low half, the reference's upload_bf16_bits,
// src/device.rs:535-549); int8 per-row (the reference's upload_int8,
// src/device.rs:550-561).
constexpr int WF32 = 0, WB16 = 1, WQ8 = 2;
constexpr int DIN_RPW = 4, GLU_RPW = 2, AQKV_RPW = 3, Z_RPW = 2;
// DeltaNet layers: units >= early_u (fp32: waves 6 and 7 of every block,
// int8: waves 4-7) have no DOUT row; they take GLU rows 0 .. (NW - early_u)
// GLU_RPW - 1 and load both of them right after DOUT's barrier, while DOUT's
// rows are summed (the other GLU rows go to units from 0 on, loaded at the
// usual time). Measured best: fp32 two waves per CU (four: +4 us per token,
// none: +9), int8 four (none: +9 us).
template <int W>
__device__ __forceinline__ constexpr int early_u() {
    return W == WF32 ? 6 * BLOCKS : 4 * BLOCKS;
}
constexpr int MIX_WAVES = VH * 8;  // 16 value columns per wave
constexpr int COMB_WAVES = NH * (HD / 4);
static_assert(DIN_RPW * NW >= DIN_ROWS && GLU_RPW * NW >= I && AQKV_RPW * NW >= AQKV_ROWS, "rows per wave");
static_assert(Z_RPW * WAVES * (BLOCKS - MIX_WAVES) >= VD && MIX_WAVES <= BLOCKS && COMB_WAVES <= NW && NKV * SMAX * QPG <= NW && SMAX % 64 == 0, "waves");
static_assert(WAVES % QPG == 0 && NKV * SMAX <= BLOCKS * (WAVES / QPG), "attention slots: QPG waves of one block each");
static_assert(4 * DIN_RPW <= WBUF && 8 * GLU_RPW <= WBUF && 4 * AQKV_RPW <= WBUF && 4 * Z_RPW <= WBUF, "buffer");
static_assert(I / 256 <= WBUF && VD / 256 <= WBUF && NH * HD / 256 <= WBUF && 8 <= WBUF && KVE <= WBUF, "buffer");
static_assert(VD / 4 == THREADS && NH == WAVES, "one thread per 4 gated values, one wave per query head");

enum : uint8_t { T_DIN, T_MIX, T_DOUT, T_GLU, T_DOWN, T_AQKV, T_ATTN, T_COMB, T_O, T_LM, T_ARG };

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

// Cross-block activations of one step, as (value, tag) pairs, per row of a
// multi-row step (a one-row step uses row 0). pml: the attention splits' (max
// score, tag), (exp sum, tag) per (query head, split); pacc: their weighted
// value sums, plain floats published by the pml pair.
struct Scratch {
    f2 x[NRMAX][H], after[NRMAX][H], proj[NRMAX][CH], z[NRMAX][VD], ab[NRMAX][2 * VH], core[NRMAX][VD];
    f2 mixed[NRMAX][QROWS], key[NRMAX][KVR], value[NRMAX][KVR], ctx[NRMAX][NH * HD], product[NRMAX][I];
    f2 pml[NRMAX][NH * SMAX * 2];
    float pacc[NRMAX][NH * SMAX * HD];
    f2 lmpart[NRMAX][NW * 4];  // (max, index, non-finite count, unused) per wave
    f2 start[BLOCKS];  // (low word of the block's start time, tag) of this launch
    unsigned lmpool[4];  // lm_head chunk counters: [epoch & 1] this launch's, the other reset for the next
};
#define SOFF(field) unsigned(offsetof(::qr::dec::Scratch, field))
// Row t of a scratch field.
#define SROW(field, t) (SOFF(field) + unsigned(t) * unsigned(sizeof(::qr::dec::Scratch::field[0])))

struct Args {
    const QrDecodeLayer* layers;
    const float* embedding;
    const float* lm_head;
    const float* final_norm;
    float* logits;
    float* picks;
    Scratch* s;
    int token, pos, vocab, nlayers;
    int emb_bf16;  // the embedding table is packed BF16 (two per word, element 2i low)
    int chain;     // 1: the token is the previous launch's argmax (picks[0]), not `token`
    float* hist;   // when set: this launch's [argmax, non-finite count] also lands here
    float* cap;    // when set (one-row steps): the step's per-layer records land here (capture layout below)
    unsigned* late;        // host-mapped flag: set when the blocks' start times spread by >= late_ticks
    unsigned late_ticks;   // (100 MHz ticks: a block that was not resident when the grid was dispatched)
    unsigned late_mask;    // launches with (epoch & late_mask) == 0 check (the check costs ~7 us)
    int snap;      // > 0: the updated DeltaNet conv and recurrent states are also written to this snapshot copy
    unsigned epoch;
    float eps;
    // multi-row steps: rows t < nrows are tokens[t] at positions pos + t;
    // rows t < snaps also write their DeltaNet states to snapshot copy snap0 + t + 1
    int nrows, snaps, snap0;
    int tokens[NRMAX];
    float rope_cs[NRMAX][ROT / 2], rope_sn[NRMAX][ROT / 2];  // cos / sin of (pos + t) / theta^(2i / rot)
};
// The layer table read through the constant address space: uniform indices
// make scalar loads, so the weight pointers stay wave-uniform (in SGPRs).
typedef const __attribute__((address_space(4))) QrDecodeLayer* LayerP;
__device__ __forceinline__ LayerP layer(const Args& a, int L) { return (LayerP)(a.layers) + L; }
// The tag of phase p's outputs in this launch.
__device__ __forceinline__ unsigned tag(const Args& a, int p) { return (a.epoch << 10) | unsigned(p + 1); }

// ---------------------------------------------------------------- memory helpers
typedef __amdgpu_buffer_rsrc_t Rs;
// Raw buffer over the whole 32-bit offset range (stride 0, dword format).
__device__ __forceinline__ Rs rsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, -1, 0x00020000);
}
// Cache policies: nt for weights (streamed once per token); sc0 sc1 +
// compiler-volatile for activations crossing blocks.
constexpr int kNT = 2;
constexpr int kSys = 1 | 16 | int(0x80000000u);

// The typed LLVM buffer intrinsics (the clang builtins return integer
// vectors, whose float reinterpretation can leave buffer entries in scratch).
__device__ f4 buffer_load_f4(Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.load.v4f32");
__device__ f2 buffer_load_f2(Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.load.v2f32");
__device__ float buffer_load_f32(Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.load.f32");
__device__ void buffer_store_f32(float v, Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.store.f32");
__device__ void buffer_store_f2(f2 v, Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.store.v2f32");
__device__ void buffer_store_f4(f4 v, Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.store.v4f32");

__device__ __forceinline__ f4 ldw(Rs r, unsigned off, unsigned soff) { return buffer_load_f4(r, off, soff, kNT); }
__device__ __forceinline__ f4 ldp4(Rs r, unsigned off, unsigned soff) { return buffer_load_f4(r, off, soff, 0); }
__device__ __forceinline__ float ldp(Rs r, unsigned off) { return buffer_load_f32(r, off, 0, 0); }
__device__ __forceinline__ void stp(Rs r, unsigned off, float v) { buffer_store_f32(v, r, off, 0, 0); }
__device__ __forceinline__ void stp4(Rs r, unsigned off, f4 v) { buffer_store_f4(v, r, off, 0, 0); }
__device__ __forceinline__ f4 ldx4(Rs r, unsigned off) { return buffer_load_f4(r, off, 0, kSys); }
__device__ __forceinline__ f2 ldx2(Rs r, unsigned off) { return buffer_load_f2(r, off, 0, kSys); }
__device__ __forceinline__ void stx(Rs r, unsigned off, float v) { buffer_store_f32(v, r, off, 0, kSys); }
__device__ __forceinline__ void stx4(Rs r, unsigned off, f4 v) { buffer_store_f4(v, r, off, 0, kSys); }
// A (value, tag) pair in one 8-byte write.
__device__ __forceinline__ void stt(Rs r, unsigned off, float v, unsigned t) {
    buffer_store_f2(f2{v, __uint_as_float(t)}, r, off, 0, kSys);
}
__device__ __forceinline__ float dot4(f4 a, f4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }
__device__ __forceinline__ float fdot4(f4 a, f4 b, float acc) {
    return fmaf(a.x, b.x, fmaf(a.y, b.y, fmaf(a.z, b.z, fmaf(a.w, b.w, acc))));
}
__device__ __forceinline__ f4 lds4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ void compiler_fence() { __atomic_signal_fence(__ATOMIC_SEQ_CST); }
// The lane index and the wave's unit index are re-materialised in every phase
// (an empty asm makes them opaque): otherwise the compiler hoists each
// phase's address arithmetic out of the phase loop and keeps all of it live
// across every phase.
__device__ __forceinline__ unsigned lane_id() {
    unsigned l = threadIdx.x & 63;
    asm volatile("" : "+v"(l));
    return l;
}
// The thread index, re-materialised the same way in multi-row kernels (NR >
// 1: there the per-thread offsets of a phase's polls kept live across all
// phases spill); one-row kernels have the registers, and are faster with the
// offsets computed once.
template <int NR>
__device__ __forceinline__ int thread_id() {
    int t = int(threadIdx.x);
    if constexpr (NR > 1) asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int opaque_uniform(int v) {
    asm volatile("" : "+s"(v));
    return v;
}

// ---------------------------------------------------------------- cross-lane steps
// DPP moves within 16-lane rows and the gfx950 row / half swaps
// (v_permlane16_swap, v_permlane32_swap): one VALU op per step, where
// __shfl_xor is a ds_bpermute through the LDS crossbar (~100+ cycles each, six
// in a row per wave sum). Each sum step adds the same pair on both lanes, so
// every lane ends with a bitwise-identical result. Whole-wave control flow
// only (a DPP read of a masked-off lane returns its stale register).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E, kRowHalfMirror = 0x141, kRowMirror = 0x140, kRowRor8 = 0x128;
// The value of lane ^ 16 (O = 16) or lane ^ 32 (O = 32).
template <int O>
__device__ __forceinline__ float lane_xor(float v) {
    static_assert(O == 16 || O == 32, "row or half swap");
    const unsigned x = __float_as_uint(v);
    const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(x, x, false, false)
                           : __builtin_amdgcn_permlane32_swap(x, x, false, false);
    // swapped: lanes of odd rows (halves) hold the partner in r[0], the others in r[1]
    return __uint_as_float((threadIdx.x & O) ? r[0] : r[1]);
}
template <int O>
__device__ __forceinline__ float xor_sum(float v) {
    const unsigned x = __float_as_uint(v);
    const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(x, x, false, false)
                           : __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);  // (even, odd) on both lanes
}
// Sum over aligned groups of W lanes (W = 16, 32 or 64).
template <int W>
__device__ __forceinline__ float lanes_sum(float v) {
    v += dpp<kQuadXor1>(v);
    v += dpp<kQuadXor2>(v);
    v += dpp<kRowHalfMirror>(v);
    v += dpp<kRowMirror>(v);
    if constexpr (W >= 32) v = xor_sum<16>(v);
    if constexpr (W >= 64) v = xor_sum<32>(v);
    return v;
}
__device__ __forceinline__ float wave_total(float v) { return lanes_sum<64>(v); }
// Sum over the four lanes of equal lane % 16.
__device__ __forceinline__ float column_sum(float v) { return xor_sum<32>(xor_sum<16>(v)); }
__device__ __forceinline__ unsigned min_u32_from(unsigned v, float other) { return min(v, __float_as_uint(other)); }
// Minimum of an unsigned over the wave (every lane gets it).
__device__ __forceinline__ unsigned wave_min_u32(unsigned v) {
    v = min_u32_from(v, dpp<kQuadXor1>(__uint_as_float(v)));
    v = min_u32_from(v, dpp<kQuadXor2>(__uint_as_float(v)));
    v = min_u32_from(v, dpp<kRowHalfMirror>(__uint_as_float(v)));
    v = min_u32_from(v, dpp<kRowMirror>(__uint_as_float(v)));
    v = min_u32_from(v, lane_xor<16>(__uint_as_float(v)));
    return min_u32_from(v, lane_xor<32>(__uint_as_float(v)));
}
__device__ __forceinline__ float wave_maximum(float v) {
    v = fmaxf(v, dpp<kQuadXor1>(v));
    v = fmaxf(v, dpp<kQuadXor2>(v));
    v = fmaxf(v, dpp<kRowHalfMirror>(v));
    v = fmaxf(v, dpp<kRowMirror>(v));
    v = fmaxf(v, lane_xor<16>(v));
    return fmaxf(v, lane_xor<32>(v));
}

// ---------------------------------------------------------------- LDS, waits
// Staged vectors of a phase: one row's [input | gated vector] (2 VD), or the
// rows of a multi-row step: NRMAX x (the DOWN input I, the DOUT input and
// gated vector H + VD, the attention's new q / k / v (NH + 2 NKV) HD).
constexpr int ACT = NRMAX * I > NRMAX * (H + VD) ? NRMAX * I : NRMAX * (H + VD);
static_assert(ACT >= 2 * VD && ACT >= NRMAX * (NH + 2 * NKV) * HD, "staging");
// Where a phase's rows sit in l.act: the layer input (row t at t H), DOUT's
// gated vector (row t at gated_off + t VD), ATTN's new q / k / v of row t at
// t (NH + 2 NKV) HD.
template <int NR>
constexpr int gated_off() { return NR == 1 ? VD : NR * H; }
constexpr int ATTN_ROW = (NH + 2 * NKV) * HD;
struct Lds {
    alignas(16) float act[2][ACT];          // staged broadcast vectors, by phase parity
    alignas(16) float nw[2][H];             // staged (1 + w) norm weights, by phase parity
    alignas(16) float wave[WAVES][2 * HD];  // wave-private scratch
    int fail;  // the earliest phase in which a lane of the block timed out (kNoFail: none)
    int token[NRMAX];  // this launch's tokens (one per row)
    int lmnext;  // the next lm_head row group of the block's range to hand out
    int lmchunk;  // the pool chunk the block streams now
    int lmctr[2];  // the next row group of that chunk, by chunk parity
    unsigned start;  // low word of this block's start time
};
constexpr int kNoFail = 0x7fffffff;

constexpr unsigned long long kTimeout = 50000000ull;  // 0.5 s at 100 MHz
// Start-time spread of a launch's blocks that marks a block as not resident
// at dispatch (a whole grid starts within a few us on an idle device).
constexpr unsigned kLateTicks = 5000;  // 50 us at 100 MHz
constexpr unsigned kLateEvery = 16;    // launches per check (power of two)

__device__ void record_failure(const Args& a, Lds& l, int p) {
    stx(rsrc(a.picks), 4, 1e30f);
    __hip_atomic_fetch_min(&l.fail, p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ int fail_phase(Lds& l) {
    return __hip_atomic_load(&l.fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ bool failed(Lds& l) { return fail_phase(l) != kNoFail; }
// Polls the two pairs at `off` until both carry tag `want` (or time-out, or
// the block has failed); returns the two values. `p`: the polling phase.
__device__ f2 wait2(const Args& a, Rs r, unsigned off, unsigned want, Lds& l, unsigned long long start, int p) {
    for (;;) {
        const f4 v = ldx4(r, off);
        if (__float_as_uint(v.y) == want && __float_as_uint(v.w) == want) return f2{v.x, v.z};
        if (wall_clock64() - start > kTimeout || failed(l)) {
            record_failure(a, l, p);
            return f2{0.f, 0.f};
        }
        __builtin_amdgcn_s_sleep(1);
    }
}
__device__ float wait1(const Args& a, Rs r, unsigned off, unsigned want, Lds& l, unsigned long long start, int p) {
    for (;;) {
        const f2 v = ldx2(r, off);
        if (__float_as_uint(v.y) == want) return v.x;
        if (wall_clock64() - start > kTimeout || failed(l)) {
            record_failure(a, l, p);
            return 0.f;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}
// Several polls at once: every load is issued before any tag is checked, so
// one round trip serves all of them when their producers are done; an entry
// not yet tagged `want` falls back to its own poll. live[k] false: skipped.
// The same, from first reads already issued into v (other loads may have been
// issued after them: they stay in flight while these are checked).
template <int N>
__device__ __forceinline__ void wait2n_from(const Args& a, Rs r, const unsigned (&off)[N], const bool (&live)[N],
                                            unsigned want, const f4 (&v)[N], f2 (&out)[N], Lds& l,
                                            unsigned long long start, int p) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
        if (!live[k]) continue;
        if (__float_as_uint(v[k].y) == want && __float_as_uint(v[k].w) == want)
            out[k] = f2{v[k].x, v[k].z};
        else
            out[k] = wait2(a, r, off[k], want, l, start, p);
    }
}
template <int N>
__device__ __forceinline__ void wait2n(const Args& a, Rs r, const unsigned (&off)[N], const bool (&live)[N],
                                       unsigned want, f2 (&out)[N], Lds& l, unsigned long long start, int p) {
    f4 v[N];
#pragma unroll
    for (int k = 0; k < N; ++k)
        if (live[k]) v[k] = ldx4(r, off[k]);
    wait2n_from<N>(a, r, off, live, want, v, out, l, start, p);
}
template <int N>
__device__ __forceinline__ void wait1n(const Args& a, Rs r, const unsigned (&off)[N], unsigned want, float (&out)[N],
                                       Lds& l, unsigned long long start, int p) {
    f2 v[N];
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = ldx2(r, off[k]);
#pragma unroll
    for (int k = 0; k < N; ++k)
        out[k] = __float_as_uint(v[k].y) == want ? v[k].x : wait1(a, r, off[k], want, l, start, p);
}
// Block barrier of phase p without a memory fence: LDS writes done
// (lgkmcnt(0)), then s_barrier; the outstanding prefetch loads stay in
// flight. Every wave of the block calls it once per phase. False when a lane
// of the block timed out in an earlier phase: every such record was made
// before its wave reached this barrier, so the block's waves agree (a record
// of phase p itself is acted on at the next barrier).
__device__ __forceinline__ bool bsync(Lds& l, int p) {
    compiler_fence();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt, expcnt not waited
    __builtin_amdgcn_s_barrier();
    compiler_fence();
    return fail_phase(l) >= p;
}

// Block barrier with no wait on memory counters. After a phase: every wave
// of the block has issued its outputs before any issues the next phase's
// loads, which would otherwise queue ahead of a late wave's output stores in
// the CU's memory pipeline.
__device__ __forceinline__ void out_barrier() {
    compiler_fence();
    __builtin_amdgcn_s_barrier();
    compiler_fence();
}

// ---------------------------------------------------------------- staging
__device__ __forceinline__ float silu(float x) { return x * sigmoidf_(x); }

// The block's 512 threads copy N (even) tagged values at scratch offset `off`
// into dst, each pair polled until tagged `want` (all of a thread's polls in
// flight together).
// `mid` runs between the first reads and their check: loads it issues (the
// second half of this phase's weights) queue behind the polls, not ahead.
struct NoMid {
    __device__ void operator()() const {}
};
// `pairs`: how many of the N / 2 pairs are polled (the rows of a multi-row
// step that take part), the rest skipped.
template <int N, int NR, class Mid = NoMid>
__device__ __forceinline__ void stage_tagged(const Args& a, Rs rs, unsigned off, unsigned want, float* dst, Lds& l,
                                             int p, Mid&& mid = Mid(), int pairs = N / 2) {
    constexpr int PAIRS = N / 2, K = (PAIRS + THREADS - 1) / THREADS;
    const unsigned long long start = wall_clock64();
    const int tid = thread_id<NR>();
    unsigned o[K];
    bool live[K];
    f4 first[K];
    f2 v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = tid + THREADS * k;
        live[k] = i < PAIRS && i < pairs;
        o[k] = off + 16u * unsigned(i);
        if (live[k]) first[k] = ldx4(rs, o[k]);
    }
    mid();
    // keep mid's loads ahead of the first check (which waits for the polls)
    asm volatile("" ::: "memory");
    wait2n_from<K>(a, rs, o, live, want, first, v, l, start, p);
#pragma unroll
    for (int k = 0; k < K; ++k)
        if (live[k]) *reinterpret_cast<f2*>(dst + 2 * (tid + THREADS * k)) = v[k];
}
// (1 + w) of an H-long norm weight into l.nw[par] (plain loads, issued before
// the tagged polls so their latency overlaps).
__device__ __forceinline__ void stage_norm(const float* w, int par, Lds& l) {
    const int t = int(threadIdx.x);
    if (t < H / 4) *reinterpret_cast<f4*>(&l.nw[par][4 * t]) = f4(1.f) + ldp4(rsrc(w), 16u * unsigned(t), 0);
}
// The layer's input residual into l.act[par]: the token's embedding row for
// layer 0 (BF16 tables only with int8 matrices, as the reference's int8
// upload keeps the embedding BF16), else x as written by phase `producer`.
template <int W, int NR, class Mid = NoMid>
__device__ __forceinline__ void stage_input(const Args& a, Rs rs, int L, int producer, int par, Lds& l, int p, int nr,
                                            Mid&& mid = Mid()) {
    if (L == 0) {
        mid();
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            if (r >= nr) break;
            const int t = int(threadIdx.x);
            float* dst = &l.act[par][r * H];
            if (W != WF32 && a.emb_bf16) {
                if (t < H / 8) {
                    const f4 wv = ldp4(rsrc(a.embedding), unsigned(l.token[r]) * unsigned(H * 2) + 16u * unsigned(t), 0);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const unsigned w = __float_as_uint(wv[j]);
                        dst[8 * t + 2 * j] = __uint_as_float(w << 16);
                        dst[8 * t + 2 * j + 1] = __uint_as_float(w & 0xffff0000u);
                    }
                }
            } else if (t < H / 4) {
                *reinterpret_cast<f4*>(dst + 4 * t) =
                    ldp4(rsrc(a.embedding), unsigned(l.token[r]) * unsigned(H * 4) + 16u * unsigned(t), 0);
            }
        }
    } else {
        stage_tagged<NR * H, NR>(a, rs, SOFF(x), tag(a, producer), l.act[par], l, p, mid, nr * (H / 2));
    }
}
// The staged H-vector in chunks times its RMSNorm and the staged (1 + w)
// (reference.h:120-126). fp32 rows: xv[v] holds elements 4 (lane + 64 v) .. +3;
// int8 rows: elements 16 lane + 4 v .. +3 (the 16 columns of the lane's
// 16-byte weight entry).
// Staged-vector element of chunk v (0..3) of `lane`: the columns a lane's
// 16-byte weight entries cover, in entry order (fp32: 4 columns per entry,
// entry v at 4 (lane + 64 v); BF16: 8 per entry, entry e at 8 (lane + 64 e),
// chunks 2e and 2e + 1 its halves; int8: one entry of 16 at 16 lane).
template <int W>
__device__ __forceinline__ constexpr unsigned xcol(unsigned lane, int v) {
    return W == WQ8    ? 16 * lane + 4 * v
           : W == WB16 ? 8 * (lane + 64 * unsigned(v >> 1)) + 4 * unsigned(v & 1)
                       : 4 * (lane + 64 * v);
}
template <int W>
__device__ __forceinline__ void normed_chunks(const Lds& l, int par, float eps, f4 (&xv)[4], int row = 0) {
    const unsigned lane = lane_id();
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        xv[v] = lds4(&l.act[par][row * H + xcol<W>(lane, v)]);
        ss += dot4(xv[v], xv[v]);
    }
    ss = wave_total(ss);
    const float r = 1.f / sqrtf(ss / float(H) + eps);
#pragma unroll
    for (int v = 0; v < 4; ++v) xv[v] = (xv[v] * r) * lds4(&l.nw[par][xcol<W>(lane, v)]);
}
// ---- capture: with a.cap set, a one-row step also writes the records of the
// engine's captured forward (src/device.rs:1748-1761 records: per layer the
// input norm, the mixer output, the residual after it, the post norm, the FFN
// product, the FFN output and the layer output) as plain stores, layer L's at
// a.cap + L CAPL, then the final norm at a.cap + nlayers CAPL.
constexpr int CAP_IN = 0, CAP_MIXED = H, CAP_AFTER = 2 * H, CAP_POST = 3 * H, CAP_PROD = 4 * H, CAP_FFN = 4 * H + I,
              CAP_OUT = 5 * H + I, CAPL = 6 * H + I;
__device__ __forceinline__ float* cap_at(const Args& a, int L, int off) { return a.cap + size_t(L) * CAPL + off; }
// A normalised vector held in normed_chunks' lane layout (one wave writes it).
template <int W>
__device__ __forceinline__ void capture_normed(float* dst, const f4 (&xv)[4]) {
    const unsigned lane = lane_id();
#pragma unroll
    for (int v = 0; v < 4; ++v) *reinterpret_cast<f4*>(dst + xcol<W>(lane, v)) = xv[v];
}
// Value e (0..3) of a word of packed int8.
__device__ __forceinline__ float q8v(unsigned w, int e) { return float(int(w << (24 - 8 * e)) >> 24); }
// 16 int8 weights (one 16-byte entry) times 16 activations.
__device__ __forceinline__ float q8dot(f4 w, const f4 (&x)[4], float acc) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned wj = __float_as_uint(w[j]);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = fmaf(q8v(wj, e), x[j][e], acc);
    }
    return acc;
}
// The two BF16 halves of a packed word (element 2i low) as fp32.
__device__ __forceinline__ float b16lo(unsigned w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float b16hi(unsigned w) { return __uint_as_float(w & 0xffff0000u); }
// 8 BF16 weights (one 16-byte entry) times 8 activations (x0: the first 4).
__device__ __forceinline__ float b16dot(f4 w, f4 x0, f4 x1, float acc) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned wj = __float_as_uint(w[j]);
        const f4& x = j < 2 ? x0 : x1;
        acc = fmaf(b16lo(wj), x[2 * (j & 1)], acc);
        acc = fmaf(b16hi(wj), x[2 * (j & 1) + 1], acc);
    }
    return acc;
}
// Row `r` of an [rows, H] matrix into wb[AT .. AT + 3]. BF16: the row's 2 KiB
// in wb[AT], wb[AT + 1] (columns 8 (lane + 64 e) .. +7 in entry e). int8
// (packed as the reference's upload_int8, src/device.rs:550-561: `rows` fp32
// scales, then the values row-major): the row's 1 KiB in wb[AT] (columns
// 16 lane .. +15) and its scale in wb[AT + 1].x.
template <int W, int AT, int AUX = kNT>
__device__ __forceinline__ void load_row_h(f4* wb, Rs m, int r, int rows) {
    const unsigned lo = 16u * lane_id();
    if constexpr (W == WQ8) {
        wb[AT] = buffer_load_f4(m, lo, unsigned(rows) * 4u + unsigned(r) * unsigned(H), AUX);
        wb[AT + 1] = f4{ldp(m, unsigned(r) * 4u), 0.f, 0.f, 0.f};
    } else if constexpr (W == WB16) {
        const unsigned row = unsigned(r) * unsigned(H * 2);
#pragma unroll
        for (int e = 0; e < 2; ++e) wb[AT + e] = buffer_load_f4(m, lo + 1024u * e, row, AUX);
    } else {
        const unsigned row = unsigned(r) * unsigned(H * 4);
#pragma unroll
        for (int v = 0; v < 4; ++v) wb[AT + v] = buffer_load_f4(m, lo + 1024u * v, row, AUX);
    }
}
// int8: scale * sum(q x), the scale after the sum (reference bridge.cpp:620-653).
template <int W, int AT>
__device__ __forceinline__ float dot_row_h(const f4* wb, const f4 (&xv)[4]) {
    float acc = 0.f;
    if constexpr (W == WQ8) return wb[AT + 1].x * wave_total(q8dot(wb[AT], xv, acc));
    if constexpr (W == WB16) return wave_total(b16dot(wb[AT + 1], xv[2], xv[3], b16dot(wb[AT], xv[0], xv[1], acc)));
#pragma unroll
    for (int v = 0; v < 4; ++v) acc = fdot4(wb[AT + v], xv[v], acc);
    return wave_total(acc);
}
// Dot of a prefetched row of K * 256 columns with the staged vector (BF16:
// K / 2 entries of 8 columns per lane, entry v at 512 v + 8 lane; int8: the
// row in ceil(K / 4) entries of 16 columns per lane, its scale after them).
template <int W, int K>
__device__ __forceinline__ float dot_row_lds(const f4* wb, const float* act) {
    const unsigned lane = lane_id();
    float acc = 0.f;
    if constexpr (W == WB16) {
        static_assert(K % 2 == 0, "BF16 rows: whole 512-column entries");
#pragma unroll
        for (int v = 0; v < K / 2; ++v) {
            const unsigned c0 = 512u * v + 8u * lane;
            acc = b16dot(wb[v], lds4(act + c0), lds4(act + c0 + 4), acc);
        }
        return wave_total(acc);
    }
    if constexpr (W == WQ8) {
        constexpr int NV = (K + 3) / 4;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const unsigned c0 = 1024u * v + 16u * lane;
            if (c0 < unsigned(K * 256)) {
                const f4 x[4] = {lds4(act + c0), lds4(act + c0 + 4), lds4(act + c0 + 8), lds4(act + c0 + 12)};
                acc = q8dot(wb[v], x, acc);
            }
        }
        return wb[NV].x * wave_total(acc);
    }
#pragma unroll
    for (int v = 0; v < K; ++v) acc = fdot4(wb[v], lds4(act + 4 * (lane + 64 * v)), acc);
    return wave_total(acc);
}

// ---------------------------------------------------------------- phases
// Each phase: every wave of the block stages (loads independent of this
// token's activations first, then the tagged inputs), one bsync, then the
// waves with work compute and store their tagged outputs. False: failed.

// ---- T_DIN: qkv | a | b rows of a DeltaNet layer (z rows: phase T_MIX), then
// the causal conv + SiLU of each qkv channel (reference.h:96-116): the wave
// computing a channel's row is the only one touching its history.
template <int W, int R, int AUX = kNT>
__device__ __forceinline__ void din_load(LayerP w, int u, f4* wb) {
    const int row = u * DIN_RPW + R;
    if (row < CH)
        load_row_h<W, 4 * R, AUX>(wb, rsrc(w->qkv), row, CH);
    else if (row < CH + VH)
        load_row_h<W, 4 * R, AUX>(wb, rsrc(w->a), row - CH, VH);
    else if (row < DIN_ROWS)
        load_row_h<W, 4 * R, AUX>(wb, rsrc(w->b), row - CH - VH, VH);
}
// Weights of the heavier phases are fetched in two parts: part 0 after the
// previous phase, part 1 after the phase's own first polls (so the polls are
// not queued behind all of it).
template <int W, int AUX = kNT>
__device__ __forceinline__ void prefetch_din(LayerP w, int u, f4* wb, int part) {
    if (part == 0) {
        din_load<W, 0, AUX>(w, u, wb);
        din_load<W, 1, AUX>(w, u, wb);
    } else {
        din_load<W, 2>(w, u, wb);
        din_load<W, 3>(w, u, wb);
    }
}
template <int W, int R>
__device__ __forceinline__ void din_row(const f4* wb, const f4 (&xv)[4], int u, float& mine) {
    if (u * DIN_RPW + R < DIN_ROWS) {
        const float acc = dot_row_h<W, 4 * R>(wb, xv);
        if (lane_id() == R) mine = acc;
    }
}
// The rows of a multi-row step run through the channel's history in order
// (the history after row r is row r's snapshot).
template <int W, int NR>
__device__ __forceinline__ bool phase_din(const Args& a, Rs rs, LayerP w, int L, int p, int u, f4* wb, Lds& l, int nr) {
    const int par = p & 1;
    const int lane = int(lane_id()), row = u * DIN_RPW + lane;
    const bool conv = lane < DIN_RPW && row < CH;
    float h0 = 0.f, h1 = 0.f, h2 = 0.f, c0 = 0.f, c1 = 0.f, c2 = 0.f, c3 = 0.f;
    const Rs hs = rsrc(w->conv_state);
    const unsigned ho = unsigned(row) * (CONVK - 1) * 4u;
    if (conv) {  // this channel's history and weights
        const Rs cw = rsrc(w->conv_w);
        const unsigned co = unsigned(row) * CONVK * 4u;
        h0 = ldp(hs, ho), h1 = ldp(hs, ho + 4), h2 = ldp(hs, ho + 8);
        c0 = ldp(cw, co), c1 = ldp(cw, co + 4), c2 = ldp(cw, co + 8), c3 = ldp(cw, co + 12);
    }
    stage_norm(w->input_norm, par, l);
    stage_input<W, NR>(a, rs, L, p - 1, par, l, p, nr, [&] { prefetch_din<W>(w, u, wb, 1); });
    if (!bsync(l, p)) return false;
    if (u * DIN_RPW >= DIN_ROWS) return true;
    float mine[NR];  // lane r: the dot product of row u * DIN_RPW + r, per step row
#pragma unroll
    for (int r = 0; r < NR; ++r) {  // every row computed (rows >= nr unused): no branch between the rows' chains
        mine[r] = 0.f;
        f4 xv[4];
        normed_chunks<W>(l, par, a.eps, xv, r);
        if (NR == 1 && a.cap && u == 0) capture_normed<W>(cap_at(a, L, CAP_IN), xv);
        din_row<W, 0>(wb, xv, u, mine[r]);
        din_row<W, 1>(wb, xv, u, mine[r]);
        din_row<W, 2>(wb, xv, u, mine[r]);
        din_row<W, 3>(wb, xv, u, mine[r]);
    }
    const unsigned t = tag(a, p);
    if (conv) {
        float hist[NR + 3];  // the history then each row's projection: row r sees hist[r .. r + 2]
        hist[0] = h0;
        hist[1] = h1;
        hist[2] = h2;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            hist[r + 3] = mine[r];
            if (r >= nr) continue;
            float sum = 0.f;
            sum += hist[r] * c0;
            sum += hist[r + 1] * c1;
            sum += hist[r + 2] * c2;
            sum += mine[r] * c3;
            // the tagged output first: stores leave in order, and a wave's stores
            // queue behind the memory traffic of its CU
            stt(rs, SROW(proj, r) + 8u * unsigned(row), silu(sum), t);
        }
        const int last = NR == 1 ? 0 : nr - 1;  // the history after the last row
        stp(hs, ho, hist[last + 1]);
        stp(hs, ho + 4, hist[last + 2]);
        stp(hs, ho + 8, hist[last + 3]);
        if (NR == 1 && a.snap > 0) {  // copy `snap` of the history (the layout of the op path's snapshots)
            const unsigned so = ho + unsigned(a.snap) * unsigned(CH * (CONVK - 1) * 4);
            stp(hs, so, h1);
            stp(hs, so + 4, h2);
            stp(hs, so + 8, mine[0]);
        }
        if (NR > 1) {
#pragma unroll
            for (int r = 0; r < NR; ++r) {  // row r's history into copy r + 1
                if (r >= nr || r >= a.snaps) break;
                const unsigned so = ho + unsigned(a.snap0 + r + 1) * unsigned(CH * (CONVK - 1) * 4);
                stp(hs, so, hist[r + 1]);
                stp(hs, so + 4, hist[r + 2]);
                stp(hs, so + 8, hist[r + 3]);
            }
        }
    } else if (lane < DIN_RPW && row < DIN_ROWS) {
#pragma unroll
        for (int r = 0; r < NR; ++r)
            if (r < nr) stt(rs, SROW(ab, r) + 8u * unsigned(row - CH), mine[r], t);
    }
    return true;
}

// ---- T_MIX: L2 q/k, gates and the gated delta rule for 16 value columns of
// one head per wave (units 0..127); silu(z), z = in_proj_z . n, on the other
// units (only silu(z) is used: the gated norm's gate, reference.h:201-207).
// z units: every wave of blocks MIX_WAVES .. BLOCKS - 1, so that no z rows
// queue ahead of the delta-rule waves' polls in their CUs (blocks 0 ..
// MIX_WAVES - 1, wave 0): 5 us per token less than z rows on units 128 ..
// 1151 of every block; -1: none
__device__ __forceinline__ int z_index(int u) {
    const int b = u % BLOCKS;
    return b >= MIX_WAVES ? (u / BLOCKS) * (BLOCKS - MIX_WAVES) + (b - MIX_WAVES) : -1;
}
template <int W, int R>
__device__ __forceinline__ void z_load(LayerP w, int u, f4* wb) {
    const int zi = z_index(u), row = zi * Z_RPW + R;
    if (zi >= 0 && row < VD) load_row_h<W, 4 * R>(wb, rsrc(w->z), row, VD);
}
template <int W>
__device__ __forceinline__ void prefetch_mix(LayerP w, int u, f4* wb) {
    if (u >= MIX_WAVES) {
        z_load<W, 0>(w, u, wb);
        z_load<W, 1>(w, u, wb);
        return;
    }
    // state S[h][i][j] (key row i, value column j), rows p*32 .. p*32+31 of column j
    const unsigned lane = lane_id();
    const int h = u >> 3, j = (u & 7) * 16 + int(lane & 15), p = int(lane >> 4);
    const Rs S = rsrc(w->recurrent);
    const unsigned base = ((unsigned(h) * DK + unsigned(p) * 32u) * DV + unsigned(j)) * 4u;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const unsigned o = base + unsigned(4 * k) * DV * 4u;
        wb[k] = f4{ldp(S, o), ldp(S, o + DV * 4u), ldp(S, o + 2u * DV * 4u), ldp(S, o + 3u * DV * 4u)};
    }
}
template <int W, int R>
__device__ __forceinline__ void z_row(Rs rs, const f4* wb, const f4 (&xv)[4], int u, unsigned t, int r, bool live) {
#pragma clang fp contract(on)
    const int zi = z_index(u), row = zi * Z_RPW + R;
    if (zi >= 0 && row < VD) {
        const float acc = dot_row_h<W, 4 * R>(wb, xv);
        if (lane_id() == 0 && live) stt(rs, SROW(z, r) + 8u * unsigned(row), silu(acc), t);
    }
}
// The delta-rule waves walk the rows of a multi-row step in order, the state
// staying in their registers (row r's state is its snapshot).
template <int W, int NR>
__device__ __forceinline__ bool phase_mix(const Args& a, Rs rs, LayerP w, int L, int p, int u, f4* wb, Lds& l,
                                          int nr) {
    // Multiply-adds contracted only within one expression: the default also
    // fuses across statements of a basic block, and the blocks of the
    // one-row and multi-row mixers differ, so their rounding would too
    // (every row must equal the one-row step bit for bit).
#pragma clang fp contract(on)
    // the z rows read the layer input and its norm weights as DIN staged them
    // (parity of phase p - 1): the block writes that buffer again only after
    // the barrier that follows this phase, so the phase needs neither a
    // staging nor a barrier of its own (a time-out of an earlier phase is
    // acted on at the next phase's barrier)
    const int par = (p - 1) & 1;
    const unsigned t = tag(a, p);
    if (u >= MIX_WAVES) {
        if (z_index(u) < 0) return true;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            f4 xv[4];
            normed_chunks<W>(l, par, a.eps, xv, r);
            z_row<W, 0>(rs, wb, xv, u, t, r, r < nr);
            z_row<W, 1>(rs, wb, xv, u, t, r, r < nr);
        }
        return true;
    }
    // the delta rule is the phase's critical path: its wave goes first on its
    // SIMD until its state is written back
    __builtin_amdgcn_s_setprio(3);
    const unsigned lane = lane_id();
    const int wave = int(threadIdx.x >> 6);
    const int h = u >> 3, cg = u & 7, pr = int(lane >> 4), j = cg * 16 + int(lane & 15);
    // convolved q and k of head h (lane: q[lane], q[lane + 64], k[lane], k[lane + 64]), v of column j
    const unsigned want = tag(a, p - 1);
    const unsigned long long start = wall_clock64();
    // every row's inputs polled at once: row r's q, k (this lane's two of
    // each), v of column j, a and b of head h
    unsigned mo[NR][7];
    f2 raw[NR][7];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const unsigned qo = SROW(proj, r) + (unsigned(h) * DK + lane) * 8u, ko = qo + KD * 8u;
        mo[r][0] = qo;
        mo[r][1] = qo + 512u;
        mo[r][2] = ko;
        mo[r][3] = ko + 512u;
        mo[r][4] = SROW(proj, r) + unsigned(2 * KD + h * DV + j) * 8u;
        mo[r][5] = SROW(ab, r) + 8u * unsigned(h);
        mo[r][6] = SROW(ab, r) + 8u * unsigned(VH + h);
        if (r < nr)
#pragma unroll
            for (int k = 0; k < 7; ++k) raw[r][k] = ldx2(rs, mo[r][k]);
    }
    // the gate parameters while the polls are in flight
    float dt = w->gates[h], alog = w->gates[VH + h];
    asm volatile("" : "+v"(dt), "+v"(alog));
    float mv[NR][7];
    bool ready = true;
#pragma unroll
    for (int r = 0; r < NR; ++r)
        if (r < nr)
#pragma unroll
            for (int k = 0; k < 7; ++k) {
                mv[r][k] = raw[r][k].x;
                ready = ready && __float_as_uint(raw[r][k].y) == want;
            }
    while (!ready) {  // every pair again in each round: one round trip serves all late ones
        if (wall_clock64() - start > kTimeout || failed(l)) {
            record_failure(a, l, p);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        ready = true;
#pragma unroll
        for (int r = 0; r < NR; ++r)
            if (r < nr) {
#pragma unroll
                for (int k = 0; k < 7; ++k) raw[r][k] = ldx2(rs, mo[r][k]);
#pragma unroll
                for (int k = 0; k < 7; ++k) {
                    mv[r][k] = raw[r][k].x;
                    ready = ready && __float_as_uint(raw[r][k].y) == want;
                }
            }
    }
    float* lw = l.wave[wave];
    const float* qq = lw + pr * 32;        // this lane's 32 key rows of q / sqrt(dk)
    const float* kk = lw + 128 + pr * 32;  // and of k
    const Rs S = rsrc(w->recurrent);
    const unsigned base = ((unsigned(h) * DK + unsigned(pr) * 32u) * DV + unsigned(j)) * 4u;
    // every row's L2 norms (reference.h:134-143) and gates (reference.h:48-60,
    // 144-148) first, with no branch between the rows' chains (rows >= nr
    // unused); then the rule walks the rows in order
    float rq[NR], rk[NR], beta_r[NR], decay_r[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float q0 = mv[r][0], q1 = mv[r][1], k0 = mv[r][2], k1 = mv[r][3], av = mv[r][5], bv = mv[r][6];
        const float sq = wave_total(q0 * q0 + q1 * q1);
        const float sk = wave_total(k0 * k0 + k1 * k1);
        rq[r] = 1.f / sqrtf(sq + 1e-6f);
        rk[r] = 1.f / sqrtf(sk + 1e-6f);
        const float log_decay = -expf(alog) * softplusf_(av + dt);
        beta_r[r] = sigmoidf_(bv);
        decay_r[r] = expf(log_decay);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        if (r >= nr) break;
        const float q0 = mv[r][0], q1 = mv[r][1], k0 = mv[r][2], k1 = mv[r][3], v = mv[r][4];
        const float sd = sqrtf(float(DK));
        lw[lane] = (q0 * rq[r]) / sd;
        lw[lane + 64] = (q1 * rq[r]) / sd;
        lw[128 + lane] = k0 * rk[r];
        lw[192 + lane] = k1 * rk[r];
        compiler_fence();
        const float beta = beta_r[r], decay = decay_r[r];
        // the rule (reference.h:149-170) on rows pr*32 .. pr*32+31 of column j, in place in wb[0..7]
        float m = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            wb[k] *= decay;
            m = fdot4(wb[k], lds4(kk + 4 * k), m);
        }
        m = column_sum(m);
        const float delta = (v - m) * beta;
        float o = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            wb[k] += lds4(kk + 4 * k) * delta;
            o = fdot4(wb[k], lds4(qq + 4 * k), o);
        }
        o = column_sum(o);
        if (pr == 0) stt(rs, SROW(core, r) + unsigned(h * DV + j) * 8u, o, t);  // the consumers' value first
        if (NR > 1 && r < a.snaps) {  // row r's state into snapshot copy snap0 + r + 1
            const unsigned sb = base + unsigned(a.snap0 + r + 1) * unsigned(VH * DK * DV * 4);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const unsigned so = sb + unsigned(4 * k) * DV * 4u;
                stp(S, so, wb[k].x);
                stp(S, so + DV * 4u, wb[k].y);
                stp(S, so + 2u * DV * 4u, wb[k].z);
                stp(S, so + 3u * DV * 4u, wb[k].w);
            }
        }
        compiler_fence();  // the next row's q / k replace this row's in the wave's scratch
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const unsigned so = base + unsigned(4 * k) * DV * 4u;
        stp(S, so, wb[k].x);
        stp(S, so + DV * 4u, wb[k].y);
        stp(S, so + 2u * DV * 4u, wb[k].z);
        stp(S, so + 3u * DV * 4u, wb[k].w);
    }
    if (NR == 1 && a.snap > 0) {  // the same state into snapshot copy `snap` (one [VH][DK][DV] state per copy)
        const unsigned sb = base + unsigned(a.snap) * unsigned(VH * DK * DV * 4);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const unsigned so = sb + unsigned(4 * k) * DV * 4u;
            stp(S, so, wb[k].x);
            stp(S, so + DV * 4u, wb[k].y);
            stp(S, so + 2u * DV * 4u, wb[k].z);
            stp(S, so + 3u * DV * 4u, wb[k].w);
        }
    }
    __builtin_amdgcn_s_setprio(0);
    return true;
}

// ---- T_DOUT: the gated RMSNorm silu(z) * RmsNorm(core) (direct weight,
// reference.h:201-207) is built once per block in LDS (thread t: elements
// 4t .. 4t+3, its head's 32 threads reduce the sum of squares; in the upper
// half of the phase's buffer, whose lower half still holds the layer input as
// DIN staged it), then out_proj row u plus that residual.
// PART -1: the whole row; 0 / 1: the first / second half of an fp32 or BF16
// row's entries (int8: part 0 is the whole row).
template <int W, int COLS, int PART = -1, int AUX = kNT>
__device__ __forceinline__ void prefetch_row(const float* m, int row, int rows, f4* wb) {
    if (row >= rows) return;
    const Rs r = rsrc(m);
    const unsigned lo = 16u * lane_id();
    if constexpr (W == WB16) {
        static_assert(COLS % 512 == 0, "BF16 rows: whole 512-column entries");
        constexpr int NB = COLS / 512, V0 = PART == 1 ? NB / 2 : 0, V1 = PART == 0 ? NB / 2 : NB;
        const unsigned ro = unsigned(row) * unsigned(COLS * 2);
#pragma unroll
        for (int v = V0; v < V1; ++v) wb[v] = buffer_load_f4(r, lo + 1024u * v, ro, AUX);
    } else if constexpr (W == WQ8) {
        if (PART == 1) return;
        constexpr int NV = (COLS + 1023) / 1024;
        const unsigned ro = unsigned(rows) * 4u + unsigned(row) * unsigned(COLS);
#pragma unroll
        for (int v = 0; v < NV; ++v)
            if (lo + 1024u * v < unsigned(COLS)) wb[v] = buffer_load_f4(r, lo + 1024u * v, ro, AUX);
        wb[NV] = f4{ldp(r, unsigned(row) * 4u), 0.f, 0.f, 0.f};
    } else {
        const unsigned ro = unsigned(row) * unsigned(COLS * 4);
        constexpr int K = COLS / 256, V0 = PART == 1 ? K / 2 : 0, V1 = PART == 0 ? K / 2 : K;
#pragma unroll
        for (int v = V0; v < V1; ++v) wb[v] = buffer_load_f4(r, lo + 1024u * v, ro, AUX);
    }
}
template <int W, int R, int AUX>
__device__ __forceinline__ void glu_load(LayerP w, int u, f4* wb);
template <int W, int NR>
__device__ __forceinline__ bool phase_dout(const Args& a, Rs rs, LayerP w, int L, int p, int u, f4* wb, Lds& l,
                                           int nr) {
    // the residual add is not fused with an int8 row's scale multiply: the
    // one-row and multi-row kernels must round it alike whatever else reads
    // the product
#pragma clang fp contract(on)
    const int par = p & 1;
    {
        const unsigned th = unsigned(thread_id<NR>());
        const f4 nw = ldp4(rsrc(w->norm_w), 16u * (th & 31), 0);
        const unsigned want = tag(a, p - 1);
        const unsigned long long start = wall_clock64();
        unsigned co[4 * NR];
        bool live[4 * NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            co[4 * r] = SROW(core, r) + 32u * th;
            co[4 * r + 1] = SROW(core, r) + 32u * th + 16u;
            co[4 * r + 2] = SROW(z, r) + 32u * th;
            co[4 * r + 3] = SROW(z, r) + 32u * th + 16u;
#pragma unroll
            for (int k = 0; k < 4; ++k) live[4 * r + k] = r < nr;
        }
        f2 cz[4 * NR];
        wait2n<4 * NR>(a, rs, co, live, want, cz, l, start, p);
#pragma unroll
        for (int r = 0; r < NR; ++r) {  // rows >= nr: unused values, no branch between the rows
            const f2 c01 = cz[4 * r], c23 = cz[4 * r + 1], z01 = cz[4 * r + 2], z23 = cz[4 * r + 3];
            const f4 core = f4{c01.x, c01.y, c23.x, c23.y}, sz = f4{z01.x, z01.y, z23.x, z23.y};
            const float ss = lanes_sum<32>(dot4(core, core));
            const float rn = 1.f / sqrtf(ss / float(DV) + a.eps);
            *reinterpret_cast<f4*>(&l.act[par][gated_off<NR>() + r * VD + 4 * th]) = sz * ((core * rn) * nw);
        }
    }
    if (!bsync(l, p)) return false;
    if (u >= H) {
        if (u >= early_u<W>()) {  // this unit's GLU rows, both parts, while DOUT's rows are summed
            glu_load<W, 0, W == WQ8 ? 0 : kNT>(w, u, wb);  // int8: part 0 stays in the memory-side cache
            glu_load<W, 1, kNT>(w, u, wb);
        }
        return true;
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float acc = dot_row_lds<W, VD / 256>(wb, l.act[par] + gated_off<NR>() + r * VD);
        const float res = l.act[par][r * H + u];  // the layer input as DIN (phase p - 2) staged it
        if (lane_id() == 0 && r < nr) stt(rs, SROW(after, r) + 8u * unsigned(u), res + acc, tag(a, p));
        if (NR == 1 && a.cap && lane_id() == 0) {
            cap_at(a, L, CAP_MIXED)[u] = acc;
            cap_at(a, L, CAP_AFTER)[u] = res + acc;
        }
    }
    return true;
}

// ---- T_GLU: product = silu(gate . n) * (up . n), n = post RMSNorm of `after`
// The first of unit u's GLU_RPW rows (dn: a DeltaNet layer).
template <int W>
__device__ __forceinline__ int glu_first(int u, bool dn) {
    if (!dn) return u * GLU_RPW;
    constexpr int E = early_u<W>(), ER = GLU_RPW * (NW - E);
    return u >= E ? (u - E) * GLU_RPW : ER + u * GLU_RPW;
}
template <int W, int R, int AUX = kNT>
__device__ __forceinline__ void glu_load(LayerP w, int u, f4* wb) {
    const int row = glu_first<W>(u, !w->attention) + R;
    if (row < I) {
        load_row_h<W, 8 * R, AUX>(wb, rsrc(w->gate), row, I);
        load_row_h<W, 8 * R + 4, AUX>(wb, rsrc(w->up), row, I);
    }
}
template <int W, int AUX = kNT>
__device__ __forceinline__ void prefetch_glu(LayerP w, int u, f4* wb, int part) {
    if (!w->attention && u >= early_u<W>()) return;  // loaded in DOUT
    if (part == 0)
        glu_load<W, 0, AUX>(w, u, wb);
    else
        glu_load<W, 1>(w, u, wb);
}
template <int W, int R>
__device__ __forceinline__ void glu_row(Rs rs, const f4* wb, const f4 (&xv)[4], int row0, unsigned t, int r,
                                        bool live = true, float* cap = nullptr) {
    const int row = row0 + R;
    if (row < I) {
        const float g = dot_row_h<W, 8 * R>(wb, xv), up = dot_row_h<W, 8 * R + 4>(wb, xv);
        if (lane_id() == 0 && live) stt(rs, SROW(product, r) + 8u * unsigned(row), silu(g) * up, t);
        if (cap && lane_id() == 0) cap[row] = silu(g) * up;
    }
}
template <int W, int NR>
__device__ __forceinline__ bool phase_glu(const Args& a, Rs rs, LayerP w, int L, int p, int u, f4* wb, Lds& l,
                                          int nr) {
    const int par = p & 1;
    stage_norm(w->post_norm, par, l);
    stage_tagged<NR * H, NR>(a, rs, SOFF(after), tag(a, p - 1), l.act[par], l, p,
                             [&] { prefetch_glu<W>(w, u, wb, 1); }, nr * (H / 2));
    if (!bsync(l, p)) return false;
    const int row0 = glu_first<W>(u, !w->attention);
    if (row0 >= I) return true;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        f4 xv[4];
        normed_chunks<W>(l, par, a.eps, xv, r);
        float* cap = nullptr;
        if (NR == 1 && a.cap) {
            if (u == 0) capture_normed<W>(cap_at(a, L, CAP_POST), xv);
            cap = cap_at(a, L, CAP_PROD);
        }
        glu_row<W, 0>(rs, wb, xv, row0, tag(a, p), r, r < nr, cap);
        glu_row<W, 1>(rs, wb, xv, row0, tag(a, p), r, r < nr, cap);
    }
    return true;
}

// One word of each 64-byte line a layer record can span (8-byte aligned
// fields at offsets 0, 56, 120, 176 of 184 bytes), read through the scalar
// cache and waited for: the next layer's first prefetch then finds its
// pointers there instead of waiting on a miss.
__device__ __forceinline__ void touch_record(LayerP w) {
    const int x0 = w->attention;
    const float* x1 = w->k;
    const float* x2 = w->a;
    const float* x3 = w->recurrent;
    asm volatile("" ::"s"(x0), "s"(x1), "s"(x2), "s"(x3));
}
// ---- T_DOWN: x = after + down . product
template <int W, int NR>
__device__ __forceinline__ bool phase_down(const Args& a, Rs rs, LayerP w, LayerP next, int L, int p, int u, f4* wb,
                                           Lds& l, int nr) {
    // the residual add is not fused with an int8 row's scale multiply: the
    // one-row and multi-row kernels must round it alike whatever else reads
    // the product
#pragma clang fp contract(on)
    const int par = p & 1;
    stage_tagged<NR * I, NR>(
        a, rs, SOFF(product), tag(a, p - 1), l.act[par], l, p,
        [&] {
            prefetch_row<W, I, 1>(w->down, u, H, wb);
            if (next) touch_record(next);
        },
        nr * (I / 2));
    if (!bsync(l, p)) return false;
    if (u >= H) return true;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float acc = dot_row_lds<W, I / 256>(wb, l.act[par] + r * I);
        const float res = l.act[par ^ 1][r * H + u];  // `after` as GLU (phase p - 1) staged it
        if (lane_id() == 0 && r < nr) stt(rs, SROW(x, r) + 8u * unsigned(u), res + acc, tag(a, p));
        if (NR == 1 && a.cap && lane_id() == 0) {
            cap_at(a, L, CAP_FFN)[u] = acc;
            cap_at(a, L, CAP_OUT)[u] = res + acc;
        }
    }
    return true;
}

// ---- T_AQKV: q ([Q | gate] per head), k, v rows of an attention layer
template <int W, int R, int AUX = kNT>
__device__ __forceinline__ void aqkv_load(LayerP w, int u, f4* wb) {
    const int row = u * AQKV_RPW + R;
    if (row < QROWS)
        load_row_h<W, 4 * R, AUX>(wb, rsrc(w->q), row, QROWS);
    else if (row < QROWS + KVR)
        load_row_h<W, 4 * R, AUX>(wb, rsrc(w->k), row - QROWS, KVR);
    else if (row < AQKV_ROWS)
        load_row_h<W, 4 * R, AUX>(wb, rsrc(w->v), row - QROWS - KVR, KVR);
}
template <int W, int AUX = kNT>
__device__ __forceinline__ void prefetch_aqkv(LayerP w, int u, f4* wb, int part) {
    if (part == 0) {
        aqkv_load<W, 0, AUX>(w, u, wb);
        aqkv_load<W, 1, AUX>(w, u, wb);
    } else {
        aqkv_load<W, 2>(w, u, wb);
    }
}
template <int W, int R>
__device__ __forceinline__ void aqkv_row(Rs rs, const f4* wb, const f4 (&xv)[4], int u, unsigned t, int r,
                                         bool live = true) {
    const int row = u * AQKV_RPW + R;
    if (row < AQKV_ROWS) {
        const float acc = dot_row_h<W, 4 * R>(wb, xv);
        if (lane_id() == 0 && live) {
            const unsigned dst = row < QROWS ? SROW(mixed, r) + 8u * unsigned(row)
                                 : row < QROWS + KVR ? SROW(key, r) + 8u * unsigned(row - QROWS)
                                                     : SROW(value, r) + 8u * unsigned(row - QROWS - KVR);
            stt(rs, dst, acc, t);
        }
    }
}
template <int W, int NR>
__device__ __forceinline__ bool phase_aqkv(const Args& a, Rs rs, LayerP w, int L, int p, int u, f4* wb, Lds& l,
                                           int nr) {
    const int par = p & 1;
    stage_norm(w->input_norm, par, l);
    stage_input<W, NR>(a, rs, L, p - 1, par, l, p, nr, [&] { prefetch_aqkv<W>(w, u, wb, 1); });
    if (!bsync(l, p)) return false;
    if (u * AQKV_RPW >= AQKV_ROWS) return true;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        f4 xv[4];
        normed_chunks<W>(l, par, a.eps, xv, r);
        if (NR == 1 && a.cap && u == 0) capture_normed<W>(cap_at(a, L, CAP_IN), xv);
        aqkv_row<W, 0>(rs, wb, xv, u, tag(a, p), r, r < nr);
        aqkv_row<W, 1>(rs, wb, xv, u, tag(a, p), r, r < nr);
        aqkv_row<W, 2>(rs, wb, xv, u, tag(a, p), r, r < nr);
    }
    return true;
}

// ---- T_ATTN: one wave per (KV head, span of positions, query head of the
// group). The QPG waves of one (KV head, span) slot sit in one block (waves
// QPG k .. QPG k + QPG - 1 of block b take slot b + BLOCKS k), so the K/V
// chunk they all read comes from HBM once and from the CU's caches for the
// others. Lane: sub = lane % 16 holds dims 64 e + 4 sub .. +3 (e < 4),
// slot = lane / 16 one of 4 positions per step, so each K / V load
// instruction reads 256 contiguous bytes of 4 rows. Caches are
// [capacity, kv_heads, head_dim].
__device__ __forceinline__ int attn_span(int len) {
    const int chunks = (len + SPAN * SMAX - 1) / (SPAN * SMAX);
    return SPAN * chunks;
}
struct AttnUnit {
    int kvh, sp, g;
    bool busy;
};
__device__ __forceinline__ AttnUnit attn_unit(int u, int splits) {
    const int block = u % BLOCKS, wave = u / BLOCKS, slot = block + BLOCKS * (wave / QPG);
    return AttnUnit{slot / splits, slot % splits, wave % QPG, slot < NKV * splits};
}
__device__ __forceinline__ void load_kv_chunk(LayerP w, int kvh, int first, int pos, f4* buf) {
    const unsigned lane = lane_id(), sub = lane & 15, slot = lane >> 4;
    const Rs rk = rsrc(w->keys), rv = rsrc(w->values);
#pragma unroll
    for (int step = 0; step < SPAN / 4; ++step) {
        const int pp = first + 4 * step + int(slot);
        if (pp < pos) {  // position pos is this step's own: patched in from LDS
            const unsigned o = ((unsigned(pp) * NKV + unsigned(kvh)) * HD + sub * 4u) * 4u;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                buf[step * 8 + e] = ldp4(rk, o + 256u * e, 0);
                buf[step * 8 + 4 + e] = ldp4(rv, o + 256u * e, 0);
            }
        }
    }
}
// The lanes whose position of the chunk at `first` is `pos` take the new
// key / value (normalised, rotated key) from LDS.
__device__ __forceinline__ void patch_new(f4* buf, const float* kn, const float* vn, int first, int pos) {
    const unsigned lane = lane_id(), sub = lane & 15, slot = lane >> 4;
#pragma unroll
    for (int step = 0; step < SPAN / 4; ++step) {
        if (first + 4 * step + int(slot) == pos) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                buf[step * 8 + e] = lds4(kn + sub * 4 + 64 * e);
                buf[step * 8 + 4 + e] = lds4(vn + sub * 4 + 64 * e);
            }
        }
    }
}
// Multi-row steps: row r (position pos + r) is split as a one-row step at
// its position would be; the rows' (KV head, split) slots are numbered row
// after row, and slot gs of the list goes to block gs % BLOCKS, wave pair
// (gs / BLOCKS) % (WAVES / QPG), round gs / (BLOCKS WAVES / QPG). False past
// the last slot.
constexpr int ATTN_PER_ROUND = BLOCKS * (WAVES / QPG);
__device__ __forceinline__ bool attn_slot(int pos, int nr, int gs, int& r, int& kvh, int& sp, int& span) {
#pragma unroll
    for (r = 0; r < NRMAX; ++r) {
        if (r >= nr) return false;
        const int len = pos + r + 1;
        span = attn_span(len);
        const int splits = (len + span - 1) / span;
        if (gs < NKV * splits) {
            kvh = gs / splits;
            sp = gs % splits;
            return true;
        }
        gs -= NKV * splits;
    }
    return false;
}
// The lanes whose position of the chunk at `first` is one of the step's new
// positions pos .. newest take that row's key / value from LDS (row q at
// rows + q ATTN_ROW).
__device__ __forceinline__ void patch_rows(f4* buf, const float* rows, int kvh, int first, int pos, int newest) {
    const unsigned lane = lane_id(), sub = lane & 15, slot = lane >> 4;
#pragma unroll
    for (int step = 0; step < SPAN / 4; ++step) {
        const int pp = first + 4 * step + int(slot);
        if (pp >= pos && pp <= newest) {
            const float* kn = rows + (pp - pos) * ATTN_ROW + NH * HD + kvh * HD;
            const float* vn = rows + (pp - pos) * ATTN_ROW + (NH + NKV) * HD + kvh * HD;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                buf[step * 8 + e] = lds4(kn + sub * 4 + 64 * e);
                buf[step * 8 + 4 + e] = lds4(vn + sub * 4 + 64 * e);
            }
        }
    }
}
template <int NR>
__device__ __forceinline__ void prefetch_attn(const Args& a, LayerP w, int u, f4* wb) {
    const int pos = a.pos;
    if (NR == 1) {
        const int len = pos + 1, span = attn_span(len), splits = (len + span - 1) / span;
        const AttnUnit au = attn_unit(u, splits);
        if (au.busy) load_kv_chunk(w, au.kvh, au.sp * span, pos, wb);
        return;
    }
    int r, kvh, sp, span;
    if (attn_slot(pos, a.nrows, (u / BLOCKS / QPG) * BLOCKS + u % BLOCKS, r, kvh, sp, span))
        load_kv_chunk(w, kvh, sp * span, pos, wb);
}
// RMSNorm (1 + w) of one head's 256 dims held 4 per lane by a whole wave,
// then rotate-half RoPE of the first 64 dims (the partner of dim d < 32 is
// d + 32, on lane + 8), into LDS (reference.h:75-95, 41-47).
__device__ __forceinline__ void norm_rope_head(f4 x, f4 wplus, const Args& a, float* out, int row = 0) {
    const unsigned lane = lane_id();
    const float ss = wave_total(dot4(x, x));
    const float r = 1.f / sqrtf(ss / float(HD) + a.eps);
    x = (x * r) * wplus;
    f4 other;  // lane ^ 8: a rotation by 8 within the 16-lane row
    other.x = dpp<kRowRor8>(x.x);
    other.y = dpp<kRowRor8>(x.y);
    other.z = dpp<kRowRor8>(x.z);
    other.w = dpp<kRowRor8>(x.w);
    if (lane < ROT / 4) {  // dims 4 lane .. 4 lane + 3 < 64
        const int i = int(4 * (lane & 7));
        const f4 cs = f4{a.rope_cs[row][i], a.rope_cs[row][i + 1], a.rope_cs[row][i + 2], a.rope_cs[row][i + 3]};
        const f4 sn = f4{a.rope_sn[row][i], a.rope_sn[row][i + 1], a.rope_sn[row][i + 2], a.rope_sn[row][i + 3]};
        x = lane < 8 ? x * cs - other * sn : x * cs + other * sn;
    }
    *reinterpret_cast<f4*>(out + 4 * lane) = x;
}
// One K/V chunk (SPAN positions from `first`, positions >= end masked) into
// the lane's running (max, sum, weighted values): both steps' scores first,
// then one rescale (reference.h:171-190, online form).
__device__ __forceinline__ void attn_chunk(const f4* kv, const f4 (&q)[4], int first, int end, float& m, float& lsum,
                                           f4 (&acc)[4]) {
    const float scale = 1.f / 16.f;  // 1 / sqrt(256)
    const int slot = int(lane_id() >> 4);
    float sc[SPAN / 4];
    bool ok[SPAN / 4];
    float mn = m;
#pragma unroll
    for (int step = 0; step < SPAN / 4; ++step) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) d = fdot4(q[e], kv[step * 8 + e], d);
        sc[step] = lanes_sum<16>(d) * scale;
        ok[step] = first + 4 * step + slot < end;
        if (ok[step]) mn = fmaxf(mn, sc[step]);
    }
    const float corr = m == -INFINITY ? 0.f : expf(m - mn);
    lsum *= corr;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] *= corr;
#pragma unroll
    for (int step = 0; step < SPAN / 4; ++step) {
        if (ok[step]) {  // a masked lane's entries hold stale registers (any bit pattern): never read
            const float pw = expf(sc[step] - mn);
            lsum += pw;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] += kv[step * 8 + 4 + e] * pw;
        }
    }
    m = mn;
}
// One (row, KV head, split, query head) unit: `pre`: its first chunk is in
// wb already (else loaded here).
template <int NR>
__device__ __forceinline__ void attn_run(const Args& a, Rs rs, LayerP w, int p, int par, Lds& l, int row, int kvh,
                                         int sp, int g, int span, bool pre, f4* wb) {
    const unsigned lane = lane_id(), sub = lane & 15, slot = lane >> 4;
    const int pos = a.pos, newest = pos + row, len = newest + 1;
    const int h = kvh * QPG + g, begin = sp * span, end = min(len, begin + span);
    const float* rows = &l.act[par][0];
    const float* kn = &l.act[par][row * ATTN_ROW + NH * HD + kvh * HD];
    const float* vn = &l.act[par][row * ATTN_ROW + (NH + NKV) * HD + kvh * HD];
    // the new positions pos .. newest that fall in [begin, end), and whether
    // this row's own position does (its unit appends it to the caches)
    const bool has_new = NR == 1 ? (pos >= begin && pos < end) : (newest >= begin && pos < end);
    const bool appends = newest >= begin && newest < end;
    if (!pre) load_kv_chunk(w, kvh, begin, pos, wb);
    if (appends && slot == 0 && g == 0) {  // one wave of the slot appends the row to the caches
        const Rs rk = rsrc(w->keys), rv = rsrc(w->values);
        const unsigned co = ((unsigned(newest) * NKV + unsigned(kvh)) * HD + sub * 4u) * 4u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            stp4(rk, co + 256u * e, lds4(kn + sub * 4 + 64 * e));
            stp4(rv, co + 256u * e, lds4(vn + sub * 4 + 64 * e));
        }
    }
    auto patch = [&](f4* buf, int first) {
        if (NR == 1)
            patch_new(buf, kn, vn, first, pos);
        else
            patch_rows(buf, rows, kvh, first, pos, newest);
    };
    if (has_new) patch(wb, begin);
    f4 q[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = lds4(&l.act[par][row * ATTN_ROW + h * HD + sub * 4 + 64 * e]);
    float m = -INFINITY, lsum = 0.f;
    f4 acc[4] = {f4(0.f), f4(0.f), f4(0.f), f4(0.f)};
    // chunks alternate between wb and nb: the next chunk's loads are in
    // flight while this one is scored
    f4 nb[KVE];
#pragma unroll 1
    for (int first = begin; first < end; first += 2 * SPAN) {
        const int c1 = first + SPAN, c2 = first + 2 * SPAN;
        if (c1 < end) load_kv_chunk(w, kvh, c1, pos, nb);
        attn_chunk(wb, q, first, end, m, lsum, acc);
        if (c1 >= end) break;
        if (has_new) patch(nb, c1);
        if (c2 < end) load_kv_chunk(w, kvh, c2, pos, wb);
        attn_chunk(nb, q, c1, end, m, lsum, acc);
        if (c2 < end && has_new) patch(wb, c2);
    }
    // merge the 4 position slots
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {
        auto exch = [o](float v) { return o == 16 ? lane_xor<16>(v) : lane_xor<32>(v); };
        const float mo = exch(m), lo = exch(lsum);
        const float mn = fmaxf(m, mo);
        const float c0 = m == -INFINITY ? 0.f : expf(m - mn), c1 = mo == -INFINITY ? 0.f : expf(mo - mn);
        lsum = lsum * c0 + lo * c1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            f4 other;
            other.x = exch(acc[e].x);
            other.y = exch(acc[e].y);
            other.z = exch(acc[e].z);
            other.w = exch(acc[e].w);
            acc[e] = acc[e] * c0 + other * c1;
        }
        m = mn;
    }
    const unsigned slotix = unsigned(h) * SMAX + unsigned(sp);
    if (slot == 0) {
        const unsigned ao = SROW(pacc, row) + (slotix * HD + sub * 4u) * 4u;
#pragma unroll
        for (int e = 0; e < 4; ++e) stx4(rs, ao + 256u * e, acc[e]);
    }
    // the weighted sums are complete in memory before their (max, sum) pair is
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    compiler_fence();
    if (lane == 0) {
        const unsigned t = tag(a, p);
        stt(rs, SROW(pml, row) + slotix * 16u, m, t);
        stt(rs, SROW(pml, row) + slotix * 16u + 8u, lsum, t);
    }
}


template <int NR>
__device__ __forceinline__ bool phase_attn(const Args& a, Rs rs, LayerP w, int p, int u, f4* wb, Lds& l, int nr) {
    const int par = p & 1;
    const int pos = a.pos, len = pos + 1, span = attn_span(len), splits = (len + span - 1) / span;
    // waves 0 .. QPG-1 hold the block's first slot (a multi-row step: every block takes part)
    const bool block_busy = NR > 1 || int(blockIdx.x) < NKV * splits;
    const int wave = int(threadIdx.x >> 6);
    const unsigned want = tag(a, p - 1);
    if (block_busy) {
        // normalised, rotated q of the 8 heads (wave h: head h), new k of the 2
        // KV heads (waves 0, 1) and their new v (waves 2, 3) into LDS, per row r
        // at r ATTN_ROW: q at + h HD, k at + NH HD + kvh HD, v at + (NH + NKV) HD + kvh HD
        const unsigned lane = lane_id();
        const Rs rn = rsrc(w->qk_norm);
        const f4 wq = f4(1.f) + ldp4(rn, 16u * lane, 0), wk = f4(1.f) + ldp4(rn, HD * 4u + 16u * lane, 0);
        const unsigned long long start = wall_clock64();
        const bool hask = wave < NKV, hasv = wave >= NKV && wave < 2 * NKV;
        unsigned qk[4 * NR];
        bool live[4 * NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const unsigned qo = SROW(mixed, r) + (unsigned(wave) * 2u * HD + 4u * lane) * 8u;
            const unsigned ko = hask   ? SROW(key, r) + (unsigned(wave) * HD + 4u * lane) * 8u
                                : hasv ? SROW(value, r) + (unsigned(wave - NKV) * HD + 4u * lane) * 8u
                                       : qo;
            qk[4 * r] = qo;
            qk[4 * r + 1] = qo + 16u;
            qk[4 * r + 2] = ko;
            qk[4 * r + 3] = ko + 16u;
            live[4 * r] = live[4 * r + 1] = r < nr;
            live[4 * r + 2] = live[4 * r + 3] = r < nr && (hask || hasv);
        }
        f2 qkv[4 * NR];
        wait2n<4 * NR>(a, rs, qk, live, want, qkv, l, start, p);
#pragma unroll
        for (int r = 0; r < NR; ++r) {  // rows >= nr: unused values
            float* rowp = &l.act[par][r * ATTN_ROW];
            norm_rope_head(f4{qkv[4 * r].x, qkv[4 * r].y, qkv[4 * r + 1].x, qkv[4 * r + 1].y}, wq, a, rowp + wave * HD, r);
            if (hask)
                norm_rope_head(f4{qkv[4 * r + 2].x, qkv[4 * r + 2].y, qkv[4 * r + 3].x, qkv[4 * r + 3].y}, wk, a,
                               rowp + NH * HD + wave * HD, r);
            if (hasv)
                *reinterpret_cast<f4*>(rowp + (NH + NKV) * HD + (wave - NKV) * HD + 4 * int(lane)) =
                    f4{qkv[4 * r + 2].x, qkv[4 * r + 2].y, qkv[4 * r + 3].x, qkv[4 * r + 3].y};
        }
    }
    if (!bsync(l, p)) return false;
    if (NR == 1) {
        const AttnUnit au = attn_unit(u, splits);
        if (au.busy) attn_run<NR>(a, rs, w, p, par, l, 0, au.kvh, au.sp, au.g, span, true, wb);
        return true;
    }
    const int block = u % BLOCKS, wv = u / BLOCKS;
    for (int round = 0;; ++round) {
        int r, kvh, sp, rspan;
        if (!attn_slot(pos, nr, round * ATTN_PER_ROUND + (wv / QPG) * BLOCKS + block, r, kvh, sp, rspan)) break;
        attn_run<NR>(a, rs, w, p, par, l, r, kvh, sp, wv % QPG, rspan, round == 0, wb);
    }
    return true;
}

// ---- T_COMB: merge the splits (log-sum-exp) and apply the sigmoid gate
// (reference.h:171-200); one wave per (head, 4 dims), lanes over splits.
constexpr int COMB_PER_LANE = SMAX / 64;
// Multi-row steps: units r COMB_WAVES .. take row r.
template <int NR>
__device__ __forceinline__ bool phase_comb(const Args& a, Rs rs, int p, int u, Lds& l, int nr) {
    static_assert(NR * COMB_WAVES <= NW, "one combine unit per wave");
    if (!bsync(l, p)) return false;
    const int row = NR == 1 ? 0 : u / COMB_WAVES;
    if (NR == 1 ? u >= COMB_WAVES : row >= nr) return true;
    const int uu = NR == 1 ? u : u % COMB_WAVES;
    const unsigned lane = lane_id();
    const int len = a.pos + row + 1, span = attn_span(len), splits = (len + span - 1) / span;
    const int h = uu / (HD / 4), c4 = uu % (HD / 4);
    const unsigned want = tag(a, p - 1);
    const unsigned long long start = wall_clock64();
    // the gate (q_proj's second half, written two phases back) in flight with the polls
    const unsigned go = SROW(mixed, row) + unsigned(h * 2 * HD + HD + 4 * c4 + int(lane & 3)) * 8u;
    const f2 gpair = ldx2(rs, go);
    float mv[COMB_PER_LANE], lv[COMB_PER_LANE];
    float mm = -INFINITY;
    bool live[COMB_PER_LANE];
    {
        unsigned po[COMB_PER_LANE];
        f2 ml[COMB_PER_LANE];
#pragma unroll
        for (int k = 0; k < COMB_PER_LANE; ++k) {
            const int s = int(lane) + 64 * k;
            live[k] = s < splits;
            po[k] = SROW(pml, row) + (unsigned(h) * SMAX + unsigned(s)) * 16u;
        }
        wait2n<COMB_PER_LANE>(a, rs, po, live, want, ml, l, start, p);
#pragma unroll
        for (int k = 0; k < COMB_PER_LANE; ++k) {
            mv[k] = live[k] ? ml[k].x : -INFINITY;
            lv[k] = live[k] ? ml[k].y : 0.f;
            mm = fmaxf(mm, mv[k]);
        }
    }
    mm = wave_maximum(mm);
    // every split's weighted sums in flight at once (dead lanes read split 0)
    f4 pv[COMB_PER_LANE];
#pragma unroll
    for (int k = 0; k < COMB_PER_LANE; ++k) {
        const unsigned ix = unsigned(h) * SMAX + (live[k] ? unsigned(lane) + 64u * k : 0u);
        pv[k] = ldx4(rs, SROW(pacc, row) + (ix * HD + unsigned(4 * c4)) * 4u);
    }
    float den = 0.f;
    f4 num = f4(0.f);
#pragma unroll
    for (int k = 0; k < COMB_PER_LANE; ++k) {
        const float wgt = live[k] ? expf(mv[k] - mm) : 0.f;
        den += lv[k] * wgt;
        num += pv[k] * wgt;
    }
    den = wave_total(den);
    num.x = wave_total(num.x);
    num.y = wave_total(num.y);
    num.z = wave_total(num.z);
    num.w = wave_total(num.w);
    if (lane < 4) {
        const float val = lane == 0 ? num.x : lane == 1 ? num.y : lane == 2 ? num.z : num.w;
        const int d = 4 * c4 + int(lane);
        const float gate = __float_as_uint(gpair.y) == tag(a, p - 2) ? gpair.x : wait1(a, rs, go, tag(a, p - 2), l, start, p);
        stt(rs, SROW(ctx, row) + unsigned(h * HD + d) * 8u, (val / den) * sigmoidf_(gate), tag(a, p));
    }
    return true;
}

// ---- T_O: after = x + o . ctx
template <int W, int NR>
__device__ __forceinline__ bool phase_o(const Args& a, Rs rs, int L, int p, int u, const f4* wb, Lds& l, int nr) {
    // the residual add is not fused with an int8 row's scale multiply: the
    // one-row and multi-row kernels must round it alike whatever else reads
    // the product
#pragma clang fp contract(on)
    const int par = p & 1;
    stage_tagged<NR * NH * HD, NR>(a, rs, SOFF(ctx), tag(a, p - 1), l.act[par], l, p, NoMid(), nr * (NH * HD / 2));
    if (!bsync(l, p)) return false;
    if (u >= H) return true;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float acc = dot_row_lds<W, NH * HD / 256>(wb, l.act[par] + r * NH * HD);
        const float res = l.act[par ^ 1][r * H + u];  // the layer input as AQKV (phase p - 3) staged it
        if (lane_id() == 0 && r < nr) stt(rs, SROW(after, r) + 8u * unsigned(u), res + acc, tag(a, p));
        if (NR == 1 && a.cap && lane_id() == 0) {
            cap_at(a, L, CAP_MIXED)[u] = acc;
            cap_at(a, L, CAP_AFTER)[u] = res + acc;
        }
    }
    return true;
}

// ---- T_LM: logits = lm_head . final RMSNorm(x); each wave streams its rows 4
// at a time with the next 4 in flight; per-wave (max, first index,
// non-finite count).
constexpr int LM_G = 4;
template <int W>
__device__ __forceinline__ void lm_load(Rs lm, int row0, int row_end, int vocab, f4* buf) {
#pragma unroll
    for (int r = 0; r < LM_G; ++r)
        if (row0 + r < row_end) {
            if constexpr (W == WQ8) {
                buf[r * 4] = ldw(lm, 16u * lane_id(), unsigned(vocab) * 4u + unsigned(row0 + r) * unsigned(H));
                buf[r * 4 + 1] = f4{ldp(lm, unsigned(row0 + r) * 4u), 0.f, 0.f, 0.f};
            } else if constexpr (W == WB16) {
                const unsigned lo = 16u * lane_id(), ro = unsigned(row0 + r) * unsigned(H * 2);
#pragma unroll
                for (int e = 0; e < 2; ++e) buf[r * 4 + e] = ldw(lm, lo + 1024u * e, ro);
            } else {
                const unsigned lo = 16u * lane_id(), ro = unsigned(row0 + r) * unsigned(H * 4);
#pragma unroll
                for (int v = 0; v < 4; ++v) buf[r * 4 + v] = ldw(lm, lo + 1024u * v, ro);
            }
        }
}
// The lm_head rows of a group are summed transposed: a lane holds V = LM_G NR
// partial dot products (value j = t LM_G + r: row r of the group against
// input row t), and the wave sums all of them at once with a butterfly whose
// first steps halve the values a lane holds (partners l ^ 32 and l ^ 16 by
// the permlane swaps, then the row mirror l ^ 15 and the half mirror l ^ 7 by
// DPP) and whose last steps are plain sums (l ^ 2, l ^ 1; and the mirrors
// when V < 16). Every value meets its partners in the same order whatever V
// is (a + b = b + a in IEEE arithmetic), so a one-row and a multi-row step sum
// each logit alike; against one wave sum per value (8 VALU operations each)
// this takes 10 operations for 4 values and 35 for 16. Afterwards lane l
// holds the total of value lm_vidx(l).
template <int V>
__device__ __forceinline__ unsigned lm_vidx(unsigned lane) {
    unsigned j = 0;
    if constexpr (V >= 2) j += (lane >> 5 & 1) * (V / 2);
    if constexpr (V >= 4) j += (lane >> 4 & 1) * (V / 4);
    if constexpr (V >= 8) j += (lane >> 3 & 1) * (V / 8);
    if constexpr (V >= 16) j += (lane >> 2 & 1) * (V / 16);
    return j;
}
// Lanes whose total is the one they report: one per value (the lowest lane
// of each group that holds it).
template <int V>
__device__ __forceinline__ bool lm_owner(unsigned lane) {
    return V >= 16 ? (lane & 3) == 0 : (lane & 15) == 0;
}
template <int V>
__device__ __forceinline__ float lm_sums(float (&v)[V]) {
    static_assert(V == 4 || V == 16, "4 or 16 values per lane");
    const unsigned lane = lane_id();
#pragma unroll
    for (int i = 0; i < V / 2; ++i) {  // l ^ 32: lanes < 32 keep values i, the others i + V / 2
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + V / 2]), false,
                                                        false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int i = 0; i < V / 4; ++i) {  // l ^ 16: even 16-lane rows keep i, odd ones i + V / 4
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + V / 4]), false,
                                                        false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    if constexpr (V >= 16) {
        const bool b3 = (lane & 8) != 0, b2 = (lane & 4) != 0;
#pragma unroll
        for (int i = 0; i < V / 8; ++i) {  // l ^ 15: lanes 0-7 of a row keep i, 8-15 i + V / 8
            const float src = b3 ? v[i] : v[i + V / 8], keep = b3 ? v[i + V / 8] : v[i];
            v[i] = keep + dpp<kRowMirror>(src);
        }
        {  // l ^ 7: lanes 0-3 of each 8 keep value 0, 4-7 value 1
            const float src = b2 ? v[0] : v[1], keep = b2 ? v[1] : v[0];
            v[0] = keep + dpp<kRowHalfMirror>(src);
        }
    } else {
        v[0] += dpp<kRowMirror>(v[0]);
        v[0] += dpp<kRowHalfMirror>(v[0]);
    }
    v[0] += dpp<kQuadXor2>(v[0]);
    v[0] += dpp<kQuadXor1>(v[0]);
    return v[0];
}
// A lane's running (max, first row of it, non-finite count) over the values it
// reports, for its input row (lm_vidx(lane) / LM_G).
struct LmBest {
    float best;
    unsigned at, bad;
};
// The LM_G rows of a group against the step's inputs (row t's logits at
// t vocab; rows >= nr computed, not stored), each lane's partial sums in the
// per-lane order of the one-row step: one-row steps with the input in
// registers; multi-row BF16 / int8 steps unpack each weight row once and take
// the NR inputs from registers (xv[t]); multi-row fp32 steps walk the inputs
// in the outer loop, each read once per group from LDS (xn: row t at t H, in
// the lane layout of normed_chunks). Then the transposed sums, the int8 row
// scale after the sum, one store per value and the lane's running maximum.
template <int W, int NR, int NX>
__device__ __forceinline__ void lm_rows(Rs lg, const f4* buf, const f4 (&xv)[NX][4], const float* xn, int row0,
                                        int row_end, int vocab, int nr, LmBest& lb) {
    constexpr int V = LM_G * NR;
    const unsigned lane = lane_id();
    float v[V];
    if constexpr (W == WF32) {
#pragma unroll
        for (int t = 0; t < NR; ++t) {
            f4 x[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) x[q] = NR == 1 ? xv[0][q] : lds4(xn + t * H + 4 * (lane + 64 * q));
#pragma unroll
            for (int r = 0; r < LM_G; ++r) {
                float acc = 0.f;
#pragma unroll
                for (int q = 0; q < 4; ++q) acc = fdot4(buf[r * 4 + q], x[q], acc);
                v[t * LM_G + r] = acc;
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < LM_G; ++r) {
            float wf[16];  // the row's 16 weights of this lane, in the one-row step's order
            if constexpr (W == WQ8) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) wf[4 * j + e] = q8v(__float_as_uint(buf[r * 4][j]), e);
            } else {
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        wf[8 * e + 2 * j] = b16lo(__float_as_uint(buf[r * 4 + e][j]));
                        wf[8 * e + 2 * j + 1] = b16hi(__float_as_uint(buf[r * 4 + e][j]));
                    }
            }
#pragma unroll
            for (int t = 0; t < NR; ++t) {
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc = fmaf(wf[4 * j + e], xv[NX == 1 ? 0 : t][j][e], acc);
                v[t * LM_G + r] = acc;
            }
        }
    }
    float acc = lm_sums<V>(v);
    const unsigned j = lm_vidx<V>(lane);
    const int r = int(j % LM_G), t = int(j / LM_G), row = row0 + r;
    if constexpr (W == WQ8) {
        const float s0 = buf[1].x, s1 = buf[5].x, s2 = buf[9].x, s3 = buf[13].x;
        acc = (r == 0 ? s0 : r == 1 ? s1 : r == 2 ? s2 : s3) * acc;
    }
    if (lm_owner<V>(lane) && row < row_end) {
        if (t < nr) stp(lg, 4u * (unsigned(t) * unsigned(vocab) + unsigned(row)), acc);
        if (!isfinite(acc)) {
            ++lb.bad;
        } else if (acc > lb.best) {
            lb.best = acc;
            lb.at = unsigned(row);
        }
    }
}
// The block's waves share the block's range of rows in groups of LM_G: each
// wave's first group is fixed (wave w: group w, prefetched), the rest are
// handed out in order by an LDS counter, so the waves of a block finish
// together (the second wave on each SIMD streams more slowly than the first).
// Every row is computed the same way whichever wave takes it.
// The first 85 % of the rows (whole groups, the same count per block) are in
// fixed block ranges; the rest is a pool of LM_CHUNK-row chunks handed to
// blocks in order by a device-wide counter once their range is done (the
// XCDs stream at different rates, by up to 20 %, and which ones are slow
// differs from GPU to GPU).
constexpr int LM_CHUNK = 64, LM_CHUNK_B16 = 128, LM_CHUNK_Q8 = 256;  // rows (BF16 / int8 rows: a half / quarter of the bytes)
__device__ __forceinline__ int lm_static_rows(int vocab) {
    return vocab / 20 * 17 / (BLOCKS * LM_G) * (BLOCKS * LM_G);
}
__device__ __forceinline__ void lm_block_range(int u, int vocab, int& first, int& last) {
    const int rb = lm_static_rows(vocab) / BLOCKS;
    first = (u % BLOCKS) * rb;
    last = first + rb;
}
template <int W>
__device__ __forceinline__ void prefetch_lm(const Args& a, int u, f4* wb) {
    int first, last;
    lm_block_range(u, a.vocab, first, last);
    lm_load<W>(rsrc(a.lm_head), first + LM_G * (u / BLOCKS), last, a.vocab, wb);
}
__device__ __forceinline__ int lm_grab(int* ctr, int first) {
    int g = 0;
    if (lane_id() == 0) g = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return first + LM_G * __builtin_amdgcn_readfirstlane(g);
}
// Rows [first, last) in groups of LM_G shared by the block's waves: wave w
// takes group w first (already in wb when `pre`), the others in order from
// the LDS counter *ctr (which starts at WAVES). Groups alternate between wb
// and nb; the counter only grows, so once a grabbed group lies past the range
// every later one does too.
template <int W, int NR, int NX>
__device__ __forceinline__ void lm_stream(Rs lm, Rs lg, const f4 (&xv)[NX][4], const float* xn, int first, int last,
                                          int vocab, int nr, int* ctr, bool pre, f4* wb, f4* nb, LmBest& lb) {
    int c0 = first + LM_G * int(threadIdx.x >> 6);
    if (!pre) lm_load<W>(lm, c0, last, vocab, wb);
    int c1 = lm_grab(ctr, first);
    lm_load<W>(lm, c1, last, vocab, nb);
    for (;;) {
        if (c0 >= last) break;
        lm_rows<W, NR, NX>(lg, wb, xv, xn, c0, last, vocab, nr, lb);
        if (c1 >= last) break;
        c0 = lm_grab(ctr, first);
        lm_load<W>(lm, c0, last, vocab, wb);
        lm_rows<W, NR, NX>(lg, nb, xv, xn, c1, last, vocab, nr, lb);
        if (c0 >= last) break;
        c1 = lm_grab(ctr, first);
        lm_load<W>(lm, c1, last, vocab, nb);
    }
}
template <int W, int NR>
__device__ __forceinline__ bool phase_lm(const Args& a, Rs rs, int p, int u, f4* wb, Lds& l, int nr) {
    const int par = p & 1;
    stage_norm(a.final_norm, par, l);
    stage_tagged<NR * H, NR>(a, rs, SOFF(x), tag(a, p - 1), l.act[par], l, p, NoMid(), nr * (H / 2));
    if (!bsync(l, p)) return false;
    // the normalised input(s): registers (one-row steps, and the rows of
    // BF16 / int8 multi-row steps), else LDS (xn, row t normalised once by
    // wave t)
    constexpr int NX = (NR == 1 || W != WF32) ? NR : 1;
    f4 xv[NX][4];
    float* xn = &l.act[par][NR * H];
    if (NR == 1) {
        normed_chunks<W>(l, par, a.eps, xv[0]);
        if (a.cap && u == 0) capture_normed<W>(cap_at(a, a.nlayers, 0), xv[0]);
    } else {
        const int wave = int(threadIdx.x >> 6);
        if (wave < NR) {
            const unsigned lane = lane_id();
            f4 x[4];
            normed_chunks<W>(l, par, a.eps, x, wave);
#pragma unroll
            for (int v = 0; v < 4; ++v)
                *reinterpret_cast<f4*>(xn + wave * H + xcol<W>(lane, v)) = x[v];
        }
        if (!bsync(l, p)) return false;
        if constexpr (W != WF32) {
            const unsigned lane = lane_id();
#pragma unroll
            for (int t = 0; t < NX; ++t)
#pragma unroll
                for (int v = 0; v < 4; ++v) xv[t][v] = lds4(xn + t * H + xcol<W>(lane, v));
        }
    }
    int first, last;
    lm_block_range(u, a.vocab, first, last);
    const Rs lm = rsrc(a.lm_head), lg = rsrc(a.logits);
    LmBest lb{-INFINITY, 0xffffffffu, 0u};
    f4 nb[4 * LM_G];
    lm_stream<W, NR, NX>(lm, lg, xv, xn, first, last, a.vocab, nr, &l.lmnext, true, wb, nb, lb);
    // then pool chunks, in increasing row order like the range (so a wave's
    // first maximum is its lowest index): thread 0 takes the block's next
    // chunk between two block barriers (the waves are done with the previous
    // chunk's counter); each take returns a larger index, so the loop ends
    constexpr int LMC = W == WQ8 ? LM_CHUNK_Q8 : W == WB16 ? LM_CHUNK_B16 : LM_CHUNK;
    const int srows = lm_static_rows(a.vocab), nchunks = (a.vocab - srows + LMC - 1) / LMC;
    for (int round = 0; round <= nchunks; ++round) {
        out_barrier();
        if (threadIdx.x == 0) {
            l.lmchunk = int(__hip_atomic_fetch_add(&a.s->lmpool[a.epoch & 1u], 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT));
            l.lmctr[round & 1] = WAVES;
        }
        out_barrier();
        const int c = __builtin_amdgcn_readfirstlane(l.lmchunk);
        if (c >= nchunks) break;
        const int cf = srows + c * LMC;
        lm_stream<W, NR, NX>(lm, lg, xv, xn, cf, min(a.vocab, cf + LMC), a.vocab, nr, &l.lmctr[round & 1], false,
                              wb, nb, lb);
    }
    // the wave's (max, first row of it, non-finite count) per input row from
    // the lanes that report its values
    const unsigned lane = lane_id(), mine = lm_vidx<LM_G * NR>(lane) / LM_G;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const bool in = mine == unsigned(r);
        const float m = wave_maximum(in ? lb.best : -INFINITY);
        const unsigned at = wave_min_u32(in && lb.best == m ? lb.at : 0xffffffffu);
        const float bad = wave_total(in ? float(lb.bad) : 0.f);
        if (lane == 0 && r < nr) {
            const unsigned o = SROW(lmpart, r) + unsigned(u) * 32u, t = tag(a, p);
            stt(rs, o, m, t);
            stt(rs, o + 8, __uint_as_float(at), t);
            stt(rs, o + 16, __uint_as_float(unsigned(bad)), t);
        }
    }
    return true;
}

// ---- T_ARG (block 0): merge the per-wave maxima (first index of the
// maximum, non-finite count; reference.h:222-230). Each of the block's
// threads polls NW / THREADS parts at once; the waves' results meet in LDS.
// Row `row` of a multi-row step (block `row` runs it).
__device__ __forceinline__ void phase_arg(const Args& a, Rs rs, int p, Lds& l, int row = 0) {
    constexpr int K = NW / THREADS;
    static_assert(NW % THREADS == 0, "argmax parts per thread");
    const unsigned lane = lane_id(), wave = threadIdx.x >> 6;
    const unsigned want = tag(a, p - 1);
    const unsigned long long start = wall_clock64();
    unsigned po[K];
    bool live[K];
    f2 vi[K], b2[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        po[k] = SROW(lmpart, row) + unsigned(int(threadIdx.x) + THREADS * k) * 32u;
        live[k] = true;
        b2[k] = ldx2(rs, po[k] + 16u);
    }
    wait2n<K>(a, rs, po, live, want, vi, l, start, p);
    float best = -INFINITY;
    unsigned at = 0xffffffffu, bad = 0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const float bk = __float_as_uint(b2[k].y) == want ? b2[k].x : wait1(a, rs, po[k] + 16u, want, l, start, p);
        bad += __float_as_uint(bk);
        const float v = vi[k].x;
        const unsigned idx = __float_as_uint(vi[k].y);
        if (v > best || (v == best && idx < at)) {
            best = v;
            at = idx;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const unsigned oi = unsigned(__shfl_xor(int(at), o, 64));
        bad += unsigned(__shfl_xor(int(bad), o, 64));
        if (ov > best || (ov == best && oi < at)) {
            best = ov;
            at = oi;
        }
    }
    if (lane == 0) {
        l.wave[wave][0] = best;
        l.wave[wave][1] = __uint_as_float(at);
        l.wave[wave][2] = __uint_as_float(bad);
    }
    if (!bsync(l, p + 1) || threadIdx.x != 0) return;
    for (int w = 1; w < WAVES; ++w) {
        const float ov = l.wave[w][0];
        const unsigned oi = __float_as_uint(l.wave[w][1]);
        bad += __float_as_uint(l.wave[w][2]);
        if (ov > best || (ov == best && oi < at)) {
            best = ov;
            at = oi;
        }
    }
    if (!failed(l)) {
        const Rs pk = rsrc(a.picks);
        stp(pk, 8u * unsigned(row), float(at));
        stp(pk, 8u * unsigned(row) + 4u, float(bad));
        if (a.hist) {
            const Rs hs = rsrc(a.hist);
            stp(hs, 0, float(at));
            stp(hs, 4, float(bad));
        }
    }
}

// ---------------------------------------------------------------- the kernel
// Part 0 of the first phase of layer L (L < nlayers).
// The weights that a phase's first polls queue behind (part 0 of DIN / AQKV /
// GLU / DOWN) are read with allocating loads in the layers of these masks,
// all other weights non-temporally: that much stays in the 256 MB memory-side
// cache from one step to the next, so those polls wait less. Measured best:
// AQKV in every attention layer and DIN in layers 0-11, 198 MB in fp32
// (ahead of the same bytes of lm_head rows, of GLU or DOWN, or of DIN in all
// layers; past ~250 MB the cache thrashes). The K/V rows are read with
// allocating loads too (24.6 KB per position in fp32): from position
// KEEP_MAX_POS on the cache is left to them (ctx 8192: 744 us per step
// instead of 763 with both).
constexpr unsigned long long kKeepDin = 0xfffull, kKeepAqkv = ~0ull, kKeepGlu = 0, kKeepDown = 0;
// int8 weights are a quarter of the bytes: part 0 of every heavy phase fits
// for many layers; layers 0-15 measured best (all 24: +7 us per token, 0-11:
// +3, 0-19: +5)
constexpr unsigned long long kKeepQ8 = 0xffffull;
// BF16 weights are half the bytes: part 0 of DIN and AQKV in every layer and
// of GLU in layers 0-5 measured best (the fp32 choice: +5 us per token; part 0
// of DOWN too: +2; int8's: +5)
constexpr unsigned long long kKeepB16Din = ~0ull, kKeepB16Aqkv = ~0ull, kKeepB16Glu = 0x3full, kKeepB16Down = 0;
// The mask of a phase's part-0 weights read with allocating loads.
template <int W>
__device__ __forceinline__ unsigned long long keep_mask(unsigned long long f32, unsigned long long b16) {
    return W == WQ8 ? kKeepQ8 : W == WB16 ? b16 : f32;
}
constexpr int KEEP_MAX_POS = 1536;
__device__ __forceinline__ bool kept(const Args& a, unsigned long long mask, int L) {
    return a.pos < KEEP_MAX_POS && ((mask >> L) & 1ull);
}
template <int W>
__device__ __forceinline__ void prefetch_layer(const Args& a, int L, int u, f4* wb) {
    const LayerP w = layer(a, L);
    if (w->attention) {
        if (kept(a, keep_mask<W>(kKeepAqkv, kKeepB16Aqkv), L))
            prefetch_aqkv<W, 0>(w, u, wb, 0);
        else
            prefetch_aqkv<W>(w, u, wb, 0);
    } else {
        if (kept(a, keep_mask<W>(kKeepDin, kKeepB16Din), L))
            prefetch_din<W, 0>(w, u, wb, 0);
        else
            prefetch_din<W>(w, u, wb, 0);
    }
}

// Residency check (the last block, after its lm_head rows): every block
// stamped its start time (tag of phase -1) on entry; a block that started
// late_ticks or more away from this one was not resident when the grid was
// dispatched (another kernel held its CU: the others' polls waited for it).
// The host-mapped flag then tells the host to launch this plan's next steps
// cooperatively, where the runtime guarantees residency. Each stamp was
// written before its block's first output, which this block has since read,
// so the stamps are visible (a tag that does not match is skipped).
__device__ __forceinline__ void check_residency(const Args& a, Rs rs, Lds& l) {
    const int t = int(threadIdx.x);
    if (t >= BLOCKS) return;
    const f2 v = ldx2(rs, SOFF(start) + 8u * unsigned(t));
    if (__float_as_uint(v.y) != tag(a, -1)) return;
    const int d = int(__float_as_uint(v.x) - l.start);
    if (unsigned(d < 0 ? -d : d) >= a.late_ticks) buffer_store_f32(__uint_as_float(1u), rsrc(a.late), 0, 0, kSys);
}

// Phase p (the tag index) runs, per DeltaNet layer, DIN MIX DOUT GLU DOWN and,
// per attention layer, AQKV ATTN COMB O GLU DOWN, then LM and ARG: per layer
// straight-line code, so the prefetch buffer flows from each phase into the
// next without a dispatch between them.
// NR > 1: a multi-row step (rows 0 .. a.nrows - 1: tokens[r] at positions
// pos + r), every phase over its rows with the weights read once; each row is
// computed exactly as a one-row step at its position (the same per-lane
// arithmetic), so row r equals that step bit for bit.
template <int W, int NR>
__global__ __launch_bounds__(THREADS, 1) void decode_kernel(Args a) {
    __shared__ Lds l;
    const int nr = NR == 1 ? 1 : a.nrows;
    // wave-uniform (readfirstlane lets the compiler keep indices and buffer
    // descriptors derived from it in SGPRs)
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int unit = wave * BLOCKS + int(blockIdx.x);  // rows spread wave-major over blocks
    const bool residency = a.late && (a.epoch & a.late_mask) == 0;
    if (threadIdx.x == 0) {
        if (residency) {
            const unsigned t0 = unsigned(wall_clock64());
            l.start = t0;
            stt(rsrc(a.s), SOFF(start) + 8u * blockIdx.x, __uint_as_float(t0), tag(a, -1));
        }
        l.fail = kNoFail;
        l.lmnext = WAVES;  // groups 0 .. WAVES - 1 are the waves' first, prefetched ones
        if (blockIdx.x == 0)  // the next launch's lm_head chunk counter (this launch uses the other)
            stx(rsrc(a.s), SOFF(lmpool) + 4u * ((a.epoch + 1u) & 1u), 0.f);
        if (NR == 1) {
            int tok = a.token;
            if (a.chain) {  // the previous launch's argmax (kernel boundary: its stores are visible)
                const float f = ldp(rsrc(a.picks), 0);
                tok = f >= 0.f && f < float(a.vocab) ? int(f) : 0;  // a bad step is reported by its own slot
            }
            l.token[0] = tok;
        } else {
#pragma unroll
            for (int r = 0; r < NR; ++r) l.token[r] = a.tokens[r];
        }
    }
    __syncthreads();
    const Rs rs = rsrc(a.s);
    f4 wb[WBUF];
    int p = 0;
    for (int L = 0; L < a.nlayers; ++L) {
        const LayerP w = layer(a, L);
        // Part 0 of the layer's first phase, issued here rather than before
        // the loop's back edge: registers with loads in flight across a back
        // edge (or a join the compiler has to reconcile) are moved there, and
        // every move waits for its load, i.e. for the whole prefetch, before
        // the layer's polls can leave. The buffer is cleared first so that no
        // earlier value has to survive into the layer.
        if (L > 0) out_barrier();
#pragma unroll
        for (int k = 0; k < WBUF; ++k) wb[k] = f4(0.f);
        prefetch_layer<W>(a, L, opaque_uniform(unit), wb);
        if (w->attention) {
            if (!phase_aqkv<W, NR>(a, rs, w, L, p, opaque_uniform(unit), wb, l, nr)) return;
            out_barrier();
            prefetch_attn<NR>(a, w, opaque_uniform(unit), wb);
            ++p;
            if (!phase_attn<NR>(a, rs, w, p, opaque_uniform(unit), wb, l, nr)) return;
            out_barrier();
            prefetch_row<W, NH * HD>(w->o, opaque_uniform(unit), H, wb);  // T_COMB reads no weights
            ++p;
            if (!phase_comb<NR>(a, rs, p, opaque_uniform(unit), l, nr)) return;
            out_barrier();
            ++p;
            if (!phase_o<W, NR>(a, rs, L, p, opaque_uniform(unit), wb, l, nr)) return;
        } else {
            if (!phase_din<W, NR>(a, rs, w, L, p, opaque_uniform(unit), wb, l, nr)) return;
            out_barrier();
            prefetch_mix<W>(w, opaque_uniform(unit), wb);
            ++p;
            if (!phase_mix<W, NR>(a, rs, w, L, p, opaque_uniform(unit), wb, l, nr)) return;
            out_barrier();
            prefetch_row<W, VD>(w->out, opaque_uniform(unit), H, wb);
            ++p;
            if (!phase_dout<W, NR>(a, rs, w, L, p, opaque_uniform(unit), wb, l, nr)) return;
        }
        out_barrier();
        if (kept(a, keep_mask<W>(kKeepGlu, kKeepB16Glu), L))
            prefetch_glu<W, 0>(w, opaque_uniform(unit), wb, 0);
        else
            prefetch_glu<W>(w, opaque_uniform(unit), wb, 0);
        ++p;
        if (!phase_glu<W, NR>(a, rs, w, L, p, opaque_uniform(unit), wb, l, nr)) return;
        out_barrier();
        if (kept(a, keep_mask<W>(kKeepDown, kKeepB16Down), L))
            prefetch_row<W, I, 0, 0>(w->down, opaque_uniform(unit), H, wb);
        else
            prefetch_row<W, I, 0>(w->down, opaque_uniform(unit), H, wb);
        ++p;
        if (!phase_down<W, NR>(a, rs, w, L + 1 < a.nlayers ? layer(a, L + 1) : nullptr, L, p, opaque_uniform(unit), wb,
                                l, nr))
            return;
        ++p;
    }
    out_barrier();
    prefetch_lm<W>(a, opaque_uniform(unit), wb);
    if (!phase_lm<W, NR>(a, rs, p, opaque_uniform(unit), wb, l, nr)) return;
    // the last block takes no argmax row: its check runs beside the argmax
    if (blockIdx.x == BLOCKS - 1 && residency) check_residency(a, rs, l);
    ++p;
    if (NR == 1) {
        if (blockIdx.x == 0) phase_arg(a, rs, p, l);
    } else if (int(blockIdx.x) < nr) {
        phase_arg(a, rs, p, l, int(blockIdx.x));
    }
}

// accept (src/device.rs:1626-1662) for every DeltaNet layer at once: the
// recurrent state and conv history of snapshot copy `rows` become the current
// ones (copy 0). Block (x, y) copies float4s x, x + gridDim.x, ... of layer
// y's two states (attention layers have none).
constexpr int ACCEPT_THREADS = 256, ACCEPT_BLOCKS = 64;
__global__ __launch_bounds__(ACCEPT_THREADS) void accept_kernel(const QrDecodeLayer* layers, int rows) {
    const QrDecodeLayer& w = layers[blockIdx.y];
    if (w.attention) return;
    constexpr int REC = VH * DK * DV / 4, CONV = CH * (CONVK - 1) / 4;  // float4s
    f4* rec = reinterpret_cast<f4*>(w.recurrent);
    f4* conv = reinterpret_cast<f4*>(w.conv_state);
    for (int i = int(blockIdx.x * ACCEPT_THREADS + threadIdx.x); i < REC; i += ACCEPT_BLOCKS * ACCEPT_THREADS)
        rec[i] = rec[size_t(rows) * REC + i];
    for (int i = int(blockIdx.x * ACCEPT_THREADS + threadIdx.x); i < CONV; i += ACCEPT_BLOCKS * ACCEPT_THREADS)
        conv[i] = conv[size_t(rows) * CONV + i];
}
static_assert((VH * DK * DV) % 4 == 0 && (CH * (CONVK - 1)) % 4 == 0, "float4 copies");

}  // namespace dec
}  // namespace qr

// ---------------------------------------------------------------- plan (host)
struct QrDecodePlan {
    qr::dec::Args args;
    QrDecodeLayer* layers = nullptr;
    qr::dec::Scratch* scratch = nullptr;  // from the device's pool
    int device = 0;
    std::vector<float> host_denom;  // theta^(2i / rot) by the host libm
    int capacity = 0;
    int snapshots = 0;          // snapshot copies behind each DeltaNet state (desc.snapshots)
    int rows = 1;               // logits / picks rows (desc.rows)
    float* logits = nullptr;    // row 0 of the logits rows ([rows, vocab])
    float* picks = nullptr;     // row 0 of the [argmax, non-finite count] rows
    int fmt = 0;  // matrix format of every layer matrix and the LM head: decode_kernel<fmt, *> (dec::WF32 / WB16 / WQ8)
    bool rows_ok = false;  // the multi-row kernel fits the device (decode_rows)
    bool cooperative = false;  // launched with hipLaunchCooperativeKernel instead of a plain launch
    unsigned* late_host = nullptr;  // host-mapped residency flag (set by a launch whose blocks started apart)
    bool auto_cooperative = true;   // a set flag switches the plan to cooperative launches
    float* hist = nullptr;  // [capacity][argmax, non-finite count] of chained steps
};

namespace qr {

const char* decode_unsupported(const QrDecodeDesc& d) {
    using namespace dec;
    if (d.hidden != H || d.intermediate != I || d.heads != NH || d.kv_heads != NKV || d.head_dim != HD ||
        d.rotary_dim != ROT || d.key_heads != KH || d.value_heads != VH || d.key_dim != DK || d.value_dim != DV ||
        d.conv_kernel != CONVK)
        return "one-launch decode is built for the Qwen3.5-0.8B geometry only";
    if (d.layers < 1 || d.layers > 64) return "one-launch decode: 1..64 layers";
    if (d.vocab < 1 || d.capacity < 1) return "one-launch decode: empty vocabulary or capacity";
    if (d.rows < 1 || d.rows > 8 || d.snapshots < 0 || d.snapshots > 7)
        return "one-launch decode: 1..8 logits rows and 0..7 snapshots";
    // every buffer offset is 32-bit: the largest matrix and cache must stay under 4 GiB
    if (double(d.vocab) * H * 4.0 >= 4294967296.0 || double(d.capacity) * NKV * HD * 4.0 >= 4294967296.0)
        return "one-launch decode: vocabulary or capacity beyond 32-bit offsets";
    if (!d.embedding || !d.final_norm || !d.logits || !d.picks || !d.layer)
        return "one-launch decode: missing buffer";
    if (d.weights != QR_DECODE_F32 && d.weights != QR_DECODE_BF16 && d.weights != QR_DECODE_INT8)
        return "one-launch decode: matrices must be all fp32, all BF16 or all int8";
    if (d.weights != QR_DECODE_F32 && !d.lm_head)
        return "one-launch decode: BF16 and int8 matrices need an LM head in the same format";
    int phases = 2;
    for (int l = 0; l < d.layers; ++l) phases += d.layer[l].attention ? 6 : 5;
    if (phases > MAXPH || phases >= 1023) return "one-launch decode: too many phases";
    return nullptr;
}

// Scratch buffers are uncached device memory (hipDeviceMallocUncached): every
// access to them is a cross-block hand-off that bypasses the L2s anyway, and on
// uncached pages a 1024-pair broadcast to all 256 blocks settles in ~1.7 us
// instead of ~2.8 us. Uncached memory that kernels have read is never handed
// back to HIP while the process runs (freeing it has been seen to corrupt
// later allocations on this platform): plans take buffers from a per-device
// pool and return them with their last launch epoch, which the next plan on
// the buffer continues, so no stale pair ever carries a tag a later launch
// expects.
namespace {
struct PooledScratch {
    qr::dec::Scratch* p;
    unsigned epoch;
};
std::mutex g_pool_mutex;
std::vector<std::pair<int, PooledScratch>> g_pool;  // (device, buffer) not in use

hipError_t scratch_acquire(int dev, hipStream_t s, qr::dec::Scratch** out, unsigned* epoch) {
    {
        std::lock_guard<std::mutex> lock(g_pool_mutex);
        for (size_t i = 0; i < g_pool.size(); ++i)
            if (g_pool[i].first == dev) {
                *out = g_pool[i].second.p;
                *epoch = g_pool[i].second.epoch;
                g_pool.erase(g_pool.begin() + long(i));
                return hipSuccess;
            }
    }
    hipError_t e = hipExtMallocWithFlags(reinterpret_cast<void**>(out), sizeof(qr::dec::Scratch),
                                         hipDeviceMallocUncached);
    if (e != hipSuccess) {
        *out = nullptr;
        return e;
    }
    *epoch = 0;
    e = hipMemsetAsync(*out, 0, sizeof(qr::dec::Scratch), s);  // tag 0: never expected
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    // A buffer whose clearing failed may hold any tag: it never enters a plan
    // or the pool (and, being uncached, is not handed back to HIP either).
    if (e != hipSuccess) *out = nullptr;
    return e;
}
void scratch_release(int dev, qr::dec::Scratch* p, unsigned epoch) {
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    g_pool.push_back({dev, PooledScratch{p, epoch}});
}
}  // namespace

// The kernel of a matrix format (dec::WF32 / WB16 / WQ8), one-row or multi-row.
void (*decode_kernel_for(int fmt, bool rows))(dec::Args) {
    using namespace dec;
    if (fmt == WQ8) return rows ? decode_kernel<WQ8, NRMAX> : decode_kernel<WQ8, 1>;
    if (fmt == WB16) return rows ? decode_kernel<WB16, NRMAX> : decode_kernel<WB16, 1>;
    return rows ? decode_kernel<WF32, NRMAX> : decode_kernel<WF32, 1>;
}

int decode_plan_create(const QrDecodeDesc& d, QrDecodePlan** out, hipStream_t s, const char** why) {
    using namespace dec;
    *out = nullptr;
    if ((*why = decode_unsupported(d))) return -1;
    int dev = 0, cus = 0, per_cu = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int fmt = d.weights == QR_DECODE_INT8 ? WQ8 : d.weights == QR_DECODE_BF16 ? WB16 : WF32;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_kernel_for(fmt, false), THREADS, 0) != hipSuccess ||
        per_cu * cus < BLOCKS) {
        *why = "one-launch decode: 256 co-resident blocks do not fit this device";
        return -1;
    }
    int rows_per_cu = 0;
    const bool rows_fit =
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&rows_per_cu, decode_kernel_for(fmt, true), THREADS, 0) ==
            hipSuccess &&
        rows_per_cu * cus >= BLOCKS;
    auto* p = new QrDecodePlan;
    std::memset(&p->args, 0, sizeof(p->args));
    p->capacity = d.capacity;
    p->snapshots = d.snapshots;
    p->rows = d.rows;
    p->logits = d.logits;
    p->picks = d.picks;
    p->fmt = fmt;
    p->rows_ok = rows_fit;
    p->device = dev;
    unsigned epoch = 0;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&p->layers), sizeof(QrDecodeLayer) * size_t(d.layers));
    if (e == hipSuccess) e = scratch_acquire(dev, s, &p->scratch, &epoch);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&p->hist), sizeof(float) * 2 * size_t(d.capacity));
    // the residency flag: pinned, mapped host memory the kernel writes and the
    // host reads before the next launch
    unsigned* late_dev = nullptr;
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&p->late_host), sizeof(unsigned), hipHostMallocMapped);
    if (e == hipSuccess) {
        *p->late_host = 0;
        e = hipHostGetDevicePointer(reinterpret_cast<void**>(&late_dev), p->late_host, 0);
    }
    p->args.epoch = epoch;  // what decode_plan_free hands back with the buffer
    // RoPE denominators theta^(2i / rot) by the host libm (the reference's
    // expression, src/attention.rs:49-50), as the op path's table
    p->host_denom.resize(ROT / 2);
    for (int i = 0; i < ROT / 2; ++i) p->host_denom[size_t(i)] = powf(d.theta, float(2 * i) / float(ROT));
    if (e == hipSuccess)
        e = hipMemcpyAsync(p->layers, d.layer, sizeof(QrDecodeLayer) * size_t(d.layers), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        decode_plan_free(p);
        *why = "one-launch decode: device allocation failed";
        return int(e);
    }
    Args& a = p->args;
    a.layers = p->layers;
    a.embedding = d.embedding;
    a.lm_head = d.lm_head ? d.lm_head : d.embedding;
    a.final_norm = d.final_norm;
    a.logits = d.logits;
    a.picks = d.picks;
    a.s = p->scratch;
    a.vocab = d.vocab;
    a.emb_bf16 = d.embedding_bf16 ? 1 : 0;
    a.eps = d.eps;
    a.epoch = epoch;
    a.late = late_dev;
    a.late_ticks = kLateTicks;
    a.late_mask = kLateEvery - 1;
    // the phase list the kernel walks (tags are phase indices): per DeltaNet
    // layer DIN MIX DOUT GLU DOWN, per attention layer AQKV ATTN COMB O GLU
    // DOWN, then LM and ARG
    a.nlayers = d.layers;
    *out = p;
    return 0;
}

bool decode_plan_is_cooperative(const QrDecodePlan* p) { return p->cooperative; }
void decode_plan_refresh(QrDecodePlan* p) {
    // a previous launch found a block that was not resident: the device is
    // shared, so residency is left to the runtime from now on
    if (!p->cooperative && p->auto_cooperative && p->late_host && __atomic_load_n(p->late_host, __ATOMIC_RELAXED) &&
        decode_plan_cooperative(p, true) != 0)
        p->auto_cooperative = false;  // no cooperative launch on this device: stay plain
}
void decode_plan_residency(QrDecodePlan* p, int ticks, bool automatic) {
    if (ticks >= 0) {
        p->args.late_ticks = unsigned(ticks);
        p->args.late_mask = ticks == 0 ? 0u : dec::kLateEvery - 1;  // the test setting checks every launch
    }
    p->auto_cooperative = automatic;
}
int decode_plan_cooperative(QrDecodePlan* p, bool on) {
    if (on) {
        int dev = 0, coop = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev);
        if (!coop) return int(hipErrorNotSupported);
    }
    p->cooperative = on;
    return 0;
}

void decode_plan_free(QrDecodePlan* p) {
    if (!p) return;
    if (p->late_host) (void)hipHostFree(p->late_host);
    if (p->layers) (void)hipFree(p->layers);
    if (p->hist) (void)hipFree(p->hist);
    if (p->scratch) scratch_release(p->device, p->scratch, p->args.epoch);
    delete p;
}

// RoPE angle pos / theta^(2i / rot) and its cos / sin on the host for row r
// (reference: src/attention.rs:49-55, the same f32 expressions).
static void set_rope(const QrDecodePlan* p, dec::Args& a, int r, int position) {
    for (int i = 0; i < dec::ROT / 2; ++i) {
        const float angle = float(position) / p->host_denom[size_t(i)];
        a.rope_cs[r][i] = cosf(angle);
        a.rope_sn[r][i] = sinf(angle);
    }
}
// Advances the launch epoch and launches the one-row or the multi-row kernel.
static int launch(QrDecodePlan* p, hipStream_t s, bool rows) {
    using namespace dec;
    Args& a = p->args;
    a.epoch = (a.epoch + 1) & 0x3fffffu;
    if (a.epoch == 0) {  // tags repeat after 2^22 steps: clear every pair first
        a.epoch = 1;
        if (hipError_t e = hipMemsetAsync(p->scratch, 0, sizeof(Scratch), s)) return int(e);
    }
    decode_plan_refresh(p);
    void* args[] = {&a};
    const void* k = reinterpret_cast<const void*>(decode_kernel_for(p->fmt, rows));
    return p->cooperative ? int(hipLaunchCooperativeKernel(k, dim3(BLOCKS), dim3(THREADS), args, 0, s))
                          : int(hipLaunchKernel(k, dim3(BLOCKS), dim3(THREADS), args, 0, s));
}

int decode_step(QrDecodePlan* p, int token, int position, int slot, hipStream_t s, int row, int snap, float* cap) {
    using namespace dec;
    Args& a = p->args;
    if (token < -1 || token >= a.vocab || position < 0 || position >= p->capacity || slot >= p->capacity ||
        row < 0 || row >= p->rows || snap < 0 || snap > p->snapshots || (row > 0 && token < 0))
        return int(hipErrorInvalidValue);
    a.logits = p->logits + size_t(row) * size_t(a.vocab);
    a.picks = p->picks + 2 * row;
    a.snap = snap;
    a.chain = token < 0 ? 1 : 0;
    a.token = token < 0 ? 0 : token;
    a.hist = slot < 0 ? nullptr : p->hist + 2 * slot;
    a.cap = cap;
    a.pos = position;
    // RoPE angle pos / theta^(2i / rot) and its cos / sin on the host
    // (reference: src/attention.rs:49-55, the same f32 expressions)
    set_rope(p, a, 0, position);
    a.nrows = 1;
    a.snaps = 0;
    a.snap0 = 0;
    return launch(p, s, false);
}

// One launch of up to NRMAX consecutive tokens (part of a verify pass): row
// r is tokens[r] at position + r, its logits in logits row first + r and
// [argmax, count] in picks row first + r; when first + r < snaps its DeltaNet
// states also go to snapshot copy first + r + 1. Each row equals the one-row
// step of its position.
int decode_rows(QrDecodePlan* p, const int* tokens, int n, int position, int first, int snaps, hipStream_t s) {
    using namespace dec;
    Args& a = p->args;
    if (!p->rows_ok) return int(hipErrorNotSupported);
    if (n < 1 || n > NRMAX || first < 0 || first + n > p->rows || position < 0 || position + n > p->capacity ||
        snaps < 0 || snaps > p->snapshots)
        return int(hipErrorInvalidValue);
    for (int r = 0; r < n; ++r)
        if (tokens[r] < 0 || tokens[r] >= a.vocab) return int(hipErrorInvalidValue);
    a.logits = p->logits + size_t(first) * size_t(a.vocab);
    a.picks = p->picks + 2 * first;
    a.snap0 = first;
    a.snap = 0;
    a.chain = 0;
    a.token = tokens[0];
    a.hist = nullptr;
    a.cap = nullptr;
    a.pos = position;
    a.nrows = n;
    a.snaps = snaps > first ? snaps - first : 0;
    for (int r = 0; r < NRMAX; ++r) {
        a.tokens[r] = r < n ? tokens[r] : 0;
        set_rope(p, a, r, position + (r < n ? r : 0));
    }
    return launch(p, s, true);
}
int decode_accept(QrDecodePlan* p, int rows, hipStream_t s) {
    using namespace dec;
    if (rows < 1 || rows > p->snapshots) return int(hipErrorInvalidValue);
    hipLaunchKernelGGL(accept_kernel, dim3(ACCEPT_BLOCKS, unsigned(p->args.nlayers)), dim3(ACCEPT_THREADS), 0, s,
                       static_cast<const QrDecodeLayer*>(p->layers), rows);
    return int(hipGetLastError());
}
size_t decode_capture_floats(const QrDecodePlan* p) {
    return size_t(p->args.nlayers) * dec::CAPL + dec::H;
}
int decode_history_clear(QrDecodePlan* p, int n, hipStream_t s) {
    if (n < 1 || n > p->capacity) return int(hipErrorInvalidValue);
    return int(hipMemsetAsync(p->hist, 0xff, sizeof(float) * 2 * size_t(n), s));  // NaN: slot never written
}
int decode_history_read(QrDecodePlan* p, int n, float* out, hipStream_t s) {
    if (n < 1 || n > p->capacity) return int(hipErrorInvalidValue);
    hipError_t e = hipMemcpyAsync(out, p->hist, sizeof(float) * 2 * size_t(n), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return int(e);
}

}  // namespace qr
