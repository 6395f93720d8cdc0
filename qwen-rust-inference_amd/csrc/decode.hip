// One decode token of the Qwen3.5-0.8B hybrid in ONE launch on gfx950
// (qr_decode_plan / qr_decode_step). It computes what the bridge's op
// sequence for one token computes (the engine's forward_body; arithmetic of
// every step as in native/rocm/reference.h), with fp32 sums in its own order.
//
// Why one launch: at batch 1 the step is a chain of ~120 dependent stages
// (each projection needs the whole previous vector). As separate kernels each
// stage pays a dispatch, a ramp-up and a drain (~2-5 us for the small
// matrices) and the step cannot approach the HBM roofline. Here 256 blocks of
// 8 waves stay resident (cooperative launch), and a stage boundary is a flag
// barrier of ~1.5 us.
//
// Structure:
//   * The phase list: per DeltaNet layer in-proj + conv, mixer (+ z rows),
//     out-proj, GLU, down; per attention layer QKV, attention, combine,
//     o-proj, GLU, down; then lm_head and argmax. All 2048 waves take part in
//     every phase; a phase's rows are spread wave-major over the blocks
//     (unit u = wave * 256 + block), so partial phases still use every CU.
//   * A wave's share of any phase's weights (and DeltaNet state / KV rows,
//     none of which depend on this token's activations) is at most 16 x 16
//     bytes per lane. Right after a wave signals phase p it issues the loads
//     of phase p + 1 into that register buffer, then waits for the barrier:
//     HBM streams the next stage while the barrier resolves.
//   * Every global access is a buffer instruction (one 32-bit lane offset, the
//     base in SGPRs). Activations crossing blocks are written and read with
//     the sc0 sc1 (system-coherent, write-through / cache-bypassing) policy;
//     a barrier is s_waitcnt on the writer's stores, then a per-block flag
//     (the last of the block's 8 waves publishes it), polled by wave 0 of each
//     block and handed to the other waves through LDS. No L2 writeback or
//     invalidate is needed and no atomic is contended.
//   * Every wait is bounded by the 100 MHz real-time counter; on a time-out
//     the wave records an error (picks[1] = 1e30, a non-finite count the
//     engine refuses) and leaves, and every other wave leaves at its next wait.
#include <cstddef>
#include <cstring>
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
constexpr int SMAX = 1024;          // attention splits per KV head
constexpr int MAXPH = 6 * 64 + 2;
constexpr int DIN_RPW = 4, GLU_RPW = 2, AQKV_RPW = 3, Z_RPW = 2;
constexpr int MIX_WAVES = VH * 8;  // 16 value columns per wave
constexpr int COMB_WAVES = NH * (HD / 4);
static_assert(DIN_RPW * NW >= DIN_ROWS && GLU_RPW * NW >= I && AQKV_RPW * NW >= AQKV_ROWS, "rows per wave");
static_assert(Z_RPW * (NW - MIX_WAVES) >= VD && COMB_WAVES <= NW && NKV * SMAX <= NW && SMAX % 64 == 0, "waves");
static_assert(4 * DIN_RPW <= WBUF && 8 * GLU_RPW <= WBUF && 4 * AQKV_RPW <= WBUF && 4 * Z_RPW <= WBUF, "buffer");
static_assert(I / 256 <= WBUF && VD / 256 <= WBUF && NH * HD / 256 <= WBUF && 8 <= WBUF, "buffer");

enum : uint8_t { T_DIN, T_MIX, T_DOUT, T_GLU, T_DOWN, T_AQKV, T_ATTN, T_COMB, T_O, T_LM, T_ARG };

typedef float f4 __attribute__((ext_vector_type(4)));

// Cross-block activations of one step. pml / pacc: the attention splits'
// (max score, exp sum) and weighted value sums per (query head, split).
struct Scratch {
    float x[H], after[H], proj[CH], z[VD], ab[2 * VH], core[VD];
    float mixed[QROWS], key[KVR], value[KVR], ctx[NH * HD], product[I];
    float pml[NH * SMAX * 2];
    float pacc[NH * SMAX * HD];
    float lmpart[NW * 3];
};
struct Sync {
    unsigned flag[BLOCKS][16];
};
#define SOFF(field) unsigned(offsetof(::qr::dec::Scratch, field))

struct Args {
    const QrDecodeLayer* layers;
    const float* embedding;
    const float* lm_head;
    const float* final_norm;
    float* logits;
    float* picks;
    const float* rope_denom;
    Scratch* s;
    Sync* sync;
    int token, pos, vocab, nphases;
    unsigned epoch;
    float eps;
    uint32_t phase[MAXPH];  // type | layer << 8
};
__device__ __forceinline__ int ptype(const Args& a, int p) { return int(a.phase[p] & 255u); }
__device__ __forceinline__ int player(const Args& a, int p) { return int(a.phase[p] >> 8); }
// The layer table read through the constant address space: uniform indices
// make scalar loads, so the weight pointers stay wave-uniform (in SGPRs).
typedef const __attribute__((address_space(4))) QrDecodeLayer* LayerP;
__device__ __forceinline__ LayerP layer(const Args& a, int L) { return (LayerP)(a.layers) + L; }

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
__device__ float buffer_load_f32(Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.load.f32");
__device__ unsigned buffer_load_u32(Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.load.i32");
__device__ void buffer_store_f32(float v, Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.store.f32");
__device__ void buffer_store_u32(unsigned v, Rs r, unsigned voff, unsigned soff, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.store.i32");

__device__ __forceinline__ f4 ldw(Rs r, unsigned off, unsigned soff) { return buffer_load_f4(r, off, soff, kNT); }
__device__ __forceinline__ f4 ldp4(Rs r, unsigned off, unsigned soff) { return buffer_load_f4(r, off, soff, 0); }
__device__ __forceinline__ float ldp(Rs r, unsigned off) { return buffer_load_f32(r, off, 0, 0); }
__device__ __forceinline__ void stp(Rs r, unsigned off, float v) { buffer_store_f32(v, r, off, 0, 0); }
__device__ __forceinline__ f4 ldx4(Rs r, unsigned off) { return buffer_load_f4(r, off, 0, kSys); }
__device__ __forceinline__ float ldx(Rs r, unsigned off) { return buffer_load_f32(r, off, 0, kSys); }
__device__ __forceinline__ void stx(Rs r, unsigned off, float v) { buffer_store_f32(v, r, off, 0, kSys); }
__device__ __forceinline__ unsigned ldu(Rs r, unsigned off) { return buffer_load_u32(r, off, 0, kSys); }
__device__ __forceinline__ void stu(Rs r, unsigned off, unsigned v) { buffer_store_u32(v, r, off, 0, kSys); }
__device__ __forceinline__ float dot4(f4 a, f4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }
__device__ __forceinline__ float fdot4(f4 a, f4 b, float acc) {
    return fmaf(a.x, b.x, fmaf(a.y, b.y, fmaf(a.z, b.z, fmaf(a.w, b.w, acc))));
}
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
__device__ __forceinline__ int opaque_uniform(int v) {
    asm volatile("" : "+s"(v));
    return v;
}

// ---------------------------------------------------------------- barrier
struct Lds {
    alignas(16) float wave[WAVES][2 * HD + ROT];  // wave-private scratch
    unsigned done[4];
    unsigned seen;
    unsigned fail;
};

constexpr unsigned long long kTimeout = 50000000ull;  // 0.5 s at 100 MHz

__device__ __forceinline__ unsigned tag(const Args& a, int p) { return (a.epoch << 10) | unsigned(p + 1); }
__device__ __forceinline__ bool reached(unsigned flag, unsigned target) { return int(flag - target) >= 0; }

__device__ void record_failure(const Args& a, Lds& l) {
    stx(rsrc(a.picks), 4, 1e30f);
    __hip_atomic_store(&l.fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Phase p's outputs of this wave are written; count the wave in, and the last
// of the block's waves publishes the block's flag.
__device__ void signal(const Args& a, Lds& l, int p) {
    compiler_fence();
    __builtin_amdgcn_s_waitcnt(0);  // every store of this wave has completed
    compiler_fence();
    if (lane_id() == 0) {
        unsigned old = __hip_atomic_fetch_add(&l.done[p & 3], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (old + 1 == unsigned(WAVES)) {
            __hip_atomic_store(&l.done[p & 3], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            stu(rsrc(a.sync), unsigned(blockIdx.x) * 64u, tag(a, p));
        }
    }
}

// Wait until phase p has completed in every block. Wave 0 of the block polls
// the block flags (4 per lane) and passes the news on in LDS.
__device__ bool wait_phase(const Args& a, Lds& l, int p, bool poller) {
    const unsigned target = tag(a, p);
    const unsigned long long start = wall_clock64();
    if (poller) {
        const Rs fl = rsrc(a.sync);
        for (;;) {
            bool ok = true;
#pragma unroll
            for (int k = 0; k < BLOCKS / 64; ++k) ok = ok && reached(ldu(fl, (lane_id() + 64u * k) * 64u), target);
            if (__all(ok)) break;
            if (wall_clock64() - start > kTimeout ||
                __hip_atomic_load(&l.fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) {
                record_failure(a, l);
                return false;
            }
        }
        if (lane_id() == 0) __hip_atomic_store(&l.seen, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
        while (!reached(__hip_atomic_load(&l.seen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP), target)) {
            __builtin_amdgcn_s_sleep(2);
            if (wall_clock64() - start > kTimeout ||
                __hip_atomic_load(&l.fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) {
                record_failure(a, l);
                return false;
            }
        }
    }
    compiler_fence();
    return true;
}

// ---------------------------------------------------------------- phase helpers
__device__ __forceinline__ float silu(float x) { return x * sigmoidf_(x); }

// The layer's input residual in chunks (element 4(lane + 64v) .. +3 in xv[v]):
// the embedding row of the token for layer 0, else the scratch x.
__device__ __forceinline__ void load_input(const Args& a, Rs rs, int L, f4 (&xv)[4]) {
    const unsigned lo = 16u * lane_id();
    if (L == 0) {
        const Rs re = rsrc(a.embedding);
        const unsigned row = unsigned(a.token) * unsigned(H * 4);
#pragma unroll
        for (int v = 0; v < 4; ++v) xv[v] = ldp4(re, lo + 1024u * v, row);
    } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) xv[v] = ldx4(rs, SOFF(x) + lo + 1024u * v);
    }
}
__device__ __forceinline__ float input_at(const Args& a, Rs rs, int L, int i) {
    if (L == 0) return ldp(rsrc(a.embedding), (unsigned(a.token) * unsigned(H) + unsigned(i)) * 4u);
    return ldx(rs, SOFF(x) + 4u * unsigned(i));
}
// RMSNorm of the H-long vector held in chunks, Qwen (1 + w) scale (reference.h:120-126).
__device__ __forceinline__ void norm_chunks(f4 (&xv)[4], const float* w, float eps) {
    const unsigned lo = 16u * lane_id();
    const Rs rw = rsrc(w);
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) ss += dot4(xv[v], xv[v]);
    ss = wave_sum(ss);
    const float r = 1.f / sqrtf(ss / float(H) + eps);
#pragma unroll
    for (int v = 0; v < 4; ++v) xv[v] = (xv[v] * r) * (f4(1.f) + ldp4(rw, lo + 1024u * v, 0));
}
// Row `r` of an [rows, H] matrix into wb[AT .. AT + 3].
template <int AT>
__device__ __forceinline__ void load_row_h(f4* wb, Rs m, int r) {
    const unsigned lo = 16u * lane_id(), row = unsigned(r) * unsigned(H * 4);
#pragma unroll
    for (int v = 0; v < 4; ++v) wb[AT + v] = ldw(m, lo + 1024u * v, row);
}
template <int AT>
__device__ __forceinline__ float dot_row_h(const f4* wb, const f4 (&xv)[4]) {
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) acc = fdot4(wb[AT + v], xv[v], acc);
    return wave_sum(acc);
}

// ---- T_DIN: qkv | a | b rows of a DeltaNet layer (z rows: phase T_MIX), then
// the causal conv + SiLU of each qkv channel (reference.h:96-116): the wave
// computing a channel's row is the only one touching its history.
template <int R>
__device__ __forceinline__ void din_load(LayerP w, int u, f4* wb) {
    const int row = u * DIN_RPW + R;
    if (row < CH)
        load_row_h<4 * R>(wb, rsrc(w->qkv), row);
    else if (row < CH + VH)
        load_row_h<4 * R>(wb, rsrc(w->a), row - CH);
    else if (row < DIN_ROWS)
        load_row_h<4 * R>(wb, rsrc(w->b), row - CH - VH);
}
__device__ __forceinline__ void prefetch_din(LayerP w, int u, f4* wb) {
    din_load<0>(w, u, wb);
    din_load<1>(w, u, wb);
    din_load<2>(w, u, wb);
    din_load<3>(w, u, wb);
}
template <int R>
__device__ __forceinline__ void din_row(const f4* wb, const f4 (&xv)[4], int u, float& mine) {
    if (u * DIN_RPW + R < DIN_ROWS) {
        const float acc = dot_row_h<4 * R>(wb, xv);
        if (lane_id() == R) mine = acc;
    }
}
__device__ void phase_din(const Args& a, Rs rs, LayerP w, int L, int u, const f4* wb) {
    if (u * DIN_RPW >= DIN_ROWS) return;
    f4 xv[4];
    load_input(a, rs, L, xv);
    norm_chunks(xv, w->input_norm, a.eps);
    float mine = 0.f;  // lane r: the dot product of row u * DIN_RPW + r
    din_row<0>(wb, xv, u, mine);
    din_row<1>(wb, xv, u, mine);
    din_row<2>(wb, xv, u, mine);
    din_row<3>(wb, xv, u, mine);
    const int lane = int(lane_id()), row = u * DIN_RPW + lane;
    if (lane < DIN_RPW && row < DIN_ROWS) {
        if (row < CH) {
            const Rs hs = rsrc(w->conv_state), cw = rsrc(w->conv_w);
            const unsigned ho = unsigned(row) * (CONVK - 1) * 4u, co = unsigned(row) * CONVK * 4u;
            const float h0 = ldp(hs, ho), h1 = ldp(hs, ho + 4), h2 = ldp(hs, ho + 8);
            float sum = 0.f;
            sum += h0 * ldp(cw, co);
            sum += h1 * ldp(cw, co + 4);
            sum += h2 * ldp(cw, co + 8);
            sum += mine * ldp(cw, co + 12);
            stp(hs, ho, h1);
            stp(hs, ho + 4, h2);
            stp(hs, ho + 8, mine);
            stx(rs, SOFF(proj) + 4u * unsigned(row), silu(sum));
        } else {
            stx(rs, SOFF(ab) + 4u * unsigned(row - CH), mine);
        }
    }
}

// ---- T_MIX: L2 q/k, gates and the gated delta rule for 16 value columns of
// one head per wave (units 0..127); z = in_proj_z . n on the other units.
template <int R>
__device__ __forceinline__ void z_load(LayerP w, int u, f4* wb) {
    const int row = (u - MIX_WAVES) * Z_RPW + R;
    if (row < VD) load_row_h<4 * R>(wb, rsrc(w->z), row);
}
__device__ __forceinline__ void prefetch_mix(LayerP w, int u, f4* wb) {
    if (u >= MIX_WAVES) {
        z_load<0>(w, u, wb);
        z_load<1>(w, u, wb);
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
template <int R>
__device__ __forceinline__ void z_row(Rs rs, const f4* wb, const f4 (&xv)[4], int u) {
    const int row = (u - MIX_WAVES) * Z_RPW + R;
    if (row < VD) {
        const float acc = dot_row_h<4 * R>(wb, xv);
        if (lane_id() == 0) stx(rs, SOFF(z) + 4u * unsigned(row), acc);
    }
}
__device__ void phase_mix(const Args& a, Rs rs, LayerP w, int L, int u, f4* wb, Lds& l) {
    if (u >= MIX_WAVES) {
        if ((u - MIX_WAVES) * Z_RPW >= VD) return;
        f4 xv[4];
        load_input(a, rs, L, xv);
        norm_chunks(xv, w->input_norm, a.eps);
        z_row<0>(rs, wb, xv, u);
        z_row<1>(rs, wb, xv, u);
        return;
    }
    const unsigned lane = lane_id();
    const int wave = int(threadIdx.x >> 6);
    const int h = u >> 3, cg = u & 7, p = int(lane >> 4), j = cg * 16 + int(lane & 15);
    // convolved q and k of head h (lane: q[lane], q[lane + 64], k[lane], k[lane + 64])
    const unsigned qo = SOFF(proj) + (unsigned(h) * DK + lane) * 4u, ko = qo + KD * 4u;
    const float q0 = ldx(rs, qo), q1 = ldx(rs, qo + 256u), k0 = ldx(rs, ko), k1 = ldx(rs, ko + 256u);
    const float v = ldx(rs, SOFF(proj) + unsigned(2 * KD + h * DV + j) * 4u);
    const float av = ldx(rs, SOFF(ab) + 4u * unsigned(h)), bv = ldx(rs, SOFF(ab) + 4u * unsigned(VH + h));
    // L2 norms (reference.h:134-143), q / sqrt(dk)
    const float sq = wave_sum(q0 * q0 + q1 * q1);
    const float sk = wave_sum(k0 * k0 + k1 * k1);
    const float rq = 1.f / sqrtf(sq + 1e-6f), rk = 1.f / sqrtf(sk + 1e-6f), sd = sqrtf(float(DK));
    float* lw = l.wave[wave];
    lw[lane] = (q0 * rq) / sd;
    lw[lane + 64] = (q1 * rq) / sd;
    lw[128 + lane] = k0 * rk;
    lw[192 + lane] = k1 * rk;
    compiler_fence();
    const float* qq = lw + p * 32;        // this lane's 32 key rows of q / sqrt(dk)
    const float* kk = lw + 128 + p * 32;  // and of k
    // gates (reference.h:48-60, 144-148)
    const float log_decay = -expf(w->gates[VH + h]) * softplusf_(av + w->gates[h]);
    const float beta = sigmoidf_(bv);
    const float decay = expf(log_decay);
    // the rule (reference.h:149-170) on rows p*32 .. p*32+31 of column j, in place in wb[0..7]
    float m = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        wb[k] *= decay;
        const f4 kv = *reinterpret_cast<const f4*>(kk + 4 * k);
        m = fdot4(wb[k], kv, m);
    }
    m += __shfl_xor(m, 16, 64);
    m += __shfl_xor(m, 32, 64);
    const float delta = (v - m) * beta;
    float o = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const f4 kv = *reinterpret_cast<const f4*>(kk + 4 * k), qv = *reinterpret_cast<const f4*>(qq + 4 * k);
        wb[k] += kv * delta;
        o = fdot4(wb[k], qv, o);
    }
    o += __shfl_xor(o, 16, 64);
    o += __shfl_xor(o, 32, 64);
    const Rs S = rsrc(w->recurrent);
    const unsigned base = ((unsigned(h) * DK + unsigned(p) * 32u) * DV + unsigned(j)) * 4u;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const unsigned so = base + unsigned(4 * k) * DV * 4u;
        stp(S, so, wb[k].x);
        stp(S, so + DV * 4u, wb[k].y);
        stp(S, so + 2u * DV * 4u, wb[k].z);
        stp(S, so + 3u * DV * 4u, wb[k].w);
    }
    if (p == 0) stx(rs, SOFF(core) + unsigned(h * DV + j) * 4u, o);
}

// ---- T_DOUT: gated RMSNorm of core with silu(z) (reference.h:201-207), then
// out_proj row u plus the residual.
template <int COLS>
__device__ __forceinline__ void prefetch_row(const float* m, int row, int rows, f4* wb) {
    if (row >= rows) return;
    const Rs r = rsrc(m);
    const unsigned lo = 16u * lane_id(), ro = unsigned(row) * unsigned(COLS * 4);
#pragma unroll
    for (int v = 0; v < COLS / 256; ++v) wb[v] = ldw(r, lo + 1024u * v, ro);
}
__device__ void phase_dout(const Args& a, Rs rs, LayerP w, int L, int u, const f4* wb) {
    if (u >= H) return;
    const unsigned lane = lane_id();
    const f4 nw = ldp4(rsrc(w->norm_w), 16u * (lane & 31), 0);  // element 4c % 128 of chunk c = lane + 64k
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const unsigned c = 16u * (lane + 64u * k);
        const f4 core = ldx4(rs, SOFF(core) + c), zz = ldx4(rs, SOFF(z) + c);
        const float ss = group_sum<32>(dot4(core, core));  // head 2k + lane / 32
        const float r = 1.f / sqrtf(ss / float(DV) + a.eps);
        const f4 g = f4{silu(zz.x), silu(zz.y), silu(zz.z), silu(zz.w)} * ((core * r) * nw);
        acc = fdot4(wb[k], g, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) stx(rs, SOFF(after) + 4u * unsigned(u), input_at(a, rs, L, u) + acc);
}

// ---- T_GLU: product = silu(gate . n) * (up . n), n = post RMSNorm of `after`
template <int R>
__device__ __forceinline__ void glu_load(LayerP w, int u, f4* wb) {
    const int row = u * GLU_RPW + R;
    if (row < I) {
        load_row_h<8 * R>(wb, rsrc(w->gate), row);
        load_row_h<8 * R + 4>(wb, rsrc(w->up), row);
    }
}
__device__ __forceinline__ void prefetch_glu(LayerP w, int u, f4* wb) {
    glu_load<0>(w, u, wb);
    glu_load<1>(w, u, wb);
}
template <int R>
__device__ __forceinline__ void glu_row(Rs rs, const f4* wb, const f4 (&xv)[4], int u) {
    const int row = u * GLU_RPW + R;
    if (row < I) {
        const float g = dot_row_h<8 * R>(wb, xv), up = dot_row_h<8 * R + 4>(wb, xv);
        if (lane_id() == 0) stx(rs, SOFF(product) + 4u * unsigned(row), silu(g) * up);
    }
}
__device__ void phase_glu(const Args& a, Rs rs, LayerP w, int u, const f4* wb) {
    if (u * GLU_RPW >= I) return;
    f4 xv[4];
    const unsigned lo = 16u * lane_id();
#pragma unroll
    for (int v = 0; v < 4; ++v) xv[v] = ldx4(rs, SOFF(after) + lo + 1024u * v);
    norm_chunks(xv, w->post_norm, a.eps);
    glu_row<0>(rs, wb, xv, u);
    glu_row<1>(rs, wb, xv, u);
}

// ---- T_DOWN: x = after + down . product
__device__ void phase_down(Rs rs, int u, const f4* wb) {
    if (u >= H) return;
    const unsigned lo = 16u * lane_id();
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < I / 256; ++v) acc = fdot4(wb[v], ldx4(rs, SOFF(product) + lo + 1024u * v), acc);
    acc = wave_sum(acc);
    if (lane_id() == 0) stx(rs, SOFF(x) + 4u * unsigned(u), ldx(rs, SOFF(after) + 4u * unsigned(u)) + acc);
}

// ---- T_AQKV: q ([Q | gate] per head), k, v rows of an attention layer
template <int R>
__device__ __forceinline__ void aqkv_load(LayerP w, int u, f4* wb) {
    const int row = u * AQKV_RPW + R;
    if (row < QROWS)
        load_row_h<4 * R>(wb, rsrc(w->q), row);
    else if (row < QROWS + KVR)
        load_row_h<4 * R>(wb, rsrc(w->k), row - QROWS);
    else if (row < AQKV_ROWS)
        load_row_h<4 * R>(wb, rsrc(w->v), row - QROWS - KVR);
}
__device__ __forceinline__ void prefetch_aqkv(LayerP w, int u, f4* wb) {
    aqkv_load<0>(w, u, wb);
    aqkv_load<1>(w, u, wb);
    aqkv_load<2>(w, u, wb);
}
template <int R>
__device__ __forceinline__ void aqkv_row(Rs rs, const f4* wb, const f4 (&xv)[4], int u) {
    const int row = u * AQKV_RPW + R;
    if (row < AQKV_ROWS) {
        const float acc = dot_row_h<4 * R>(wb, xv);
        if (lane_id() == 0) {
            const unsigned dst = row < QROWS ? SOFF(mixed) + 4u * unsigned(row)
                                 : row < QROWS + KVR ? SOFF(key) + 4u * unsigned(row - QROWS)
                                                     : SOFF(value) + 4u * unsigned(row - QROWS - KVR);
            stx(rs, dst, acc);
        }
    }
}
__device__ void phase_aqkv(const Args& a, Rs rs, LayerP w, int L, int u, const f4* wb) {
    if (u * AQKV_RPW >= AQKV_ROWS) return;
    f4 xv[4];
    load_input(a, rs, L, xv);
    norm_chunks(xv, w->input_norm, a.eps);
    aqkv_row<0>(rs, wb, xv, u);
    aqkv_row<1>(rs, wb, xv, u);
    aqkv_row<2>(rs, wb, xv, u);
}

// ---- T_ATTN: one wave per (KV head, span of positions); the 4 query heads of
// the group share every K/V read. Lane: sub = lane % 16 holds dims
// 16 sub .. 16 sub + 15, slot = lane / 16 one of 4 positions per step.
// Caches are [capacity, kv_heads, head_dim].
__device__ __forceinline__ int attn_span(int len) {
    const int chunks = (len + SPAN * SMAX - 1) / (SPAN * SMAX);
    return SPAN * chunks;
}
__device__ __forceinline__ void load_kv_chunk(LayerP w, int kvh, int first, int pos, f4* buf) {
    const unsigned lane = lane_id(), sub = lane & 15, slot = lane >> 4;
    const Rs rk = rsrc(w->keys), rv = rsrc(w->values);
#pragma unroll
    for (int step = 0; step < SPAN / 4; ++step) {
        const int pp = first + 4 * step + int(slot);
        if (pp < pos) {  // position pos is this step's own: patched in from LDS
            const unsigned o = ((unsigned(pp) * NKV + unsigned(kvh)) * HD + sub * 16u) * 4u;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                buf[step * 8 + e] = ldw(rk, o + 16u * e, 0);
                buf[step * 8 + 4 + e] = ldw(rv, o + 16u * e, 0);
            }
        }
    }
}
// The lanes whose position of the chunk at `first` is `pos` take the new
// key / value (normalised, rotated) from the wave's LDS.
__device__ __forceinline__ void patch_new(f4* buf, const float* lw, int first, int pos) {
    const unsigned lane = lane_id(), sub = lane & 15, slot = lane >> 4;
#pragma unroll
    for (int step = 0; step < SPAN / 4; ++step) {
        if (first + 4 * step + int(slot) == pos) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                buf[step * 8 + e] = *reinterpret_cast<const f4*>(lw + sub * 16 + 4 * e);
                buf[step * 8 + 4 + e] = *reinterpret_cast<const f4*>(lw + HD + sub * 16 + 4 * e);
            }
        }
    }
}
__device__ __forceinline__ void prefetch_attn(LayerP w, int u, int pos, f4* wb) {
    const int len = pos + 1, span = attn_span(len), splits = (len + span - 1) / span;
    if (u >= NKV * splits) return;
    load_kv_chunk(w, u / splits, (u % splits) * span, pos, wb);
}
// cos / sin of the RoPE angles pos / theta^(2i / rot), i < rot / 2, one per
// lane, into trig[0, 32) / trig[32, 64) (reference.h:41-47).
__device__ __forceinline__ void rope_trig(float* trig, const float* denom, int pos) {
    const unsigned lane = lane_id();
    if (lane < ROT / 2) {
        const float angle = float(pos) / denom[lane];
        trig[lane] = cosf(angle);
        trig[ROT / 2 + lane] = sinf(angle);
    }
    compiler_fence();
}
// RMSNorm (1 + w) over the 256 dims spread as 16 per lane over 16 lanes, then
// rotate-half RoPE of the first 64 dims (partner dims 32 apart live on
// lane ^ 2). Reference: reference.h:75-95.
__device__ __forceinline__ void norm_rope16(float (&x)[16], const float* w, const float* trig, float eps) {
    const unsigned sub = lane_id() & 15;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) ss += x[e] * x[e];
    ss = group_sum<16>(ss);
    const float r = 1.f / sqrtf(ss / float(HD) + eps);
    const Rs rw = rsrc(w);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const f4 wv = ldp4(rw, 64u * sub + 16u * e, 0);
        x[4 * e] = (x[4 * e] * r) * (1.f + wv.x);
        x[4 * e + 1] = (x[4 * e + 1] * r) * (1.f + wv.y);
        x[4 * e + 2] = (x[4 * e + 2] * r) * (1.f + wv.z);
        x[4 * e + 3] = (x[4 * e + 3] * r) * (1.f + wv.w);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const float other = __shfl_xor(x[e], 2, 64);
        if (sub < 4) {
            const int i = int(sub & 1) * 16 + e;
            const float cs = trig[i], sn = trig[ROT / 2 + i];
            x[e] = sub < 2 ? x[e] * cs - other * sn : x[e] * cs + other * sn;
        }
    }
}
__device__ void phase_attn(const Args& a, Rs rs, LayerP w, int u, f4* wb, Lds& l) {
    const int pos = a.pos, len = pos + 1, span = attn_span(len), splits = (len + span - 1) / span;
    if (u >= NKV * splits) return;
    const unsigned lane = lane_id(), sub = lane & 15, slot = lane >> 4;
    const int wave = int(threadIdx.x >> 6);
    const int kvh = u / splits, sp = u % splits, begin = sp * span, end = min(len, begin + span);
    float* lw = l.wave[wave];  // [0, HD): the new key, [HD, 2 HD): the new value
    float* trig = lw + 2 * HD;
    rope_trig(trig, a.rope_denom, pos);
    const bool has_new = pos >= begin && pos < end;
    if (has_new) {
        float kn[16];
        const unsigned ko = SOFF(key) + (unsigned(kvh) * HD + sub * 16u) * 4u;
#pragma unroll
        for (int e = 0; e < 16; ++e) kn[e] = ldx(rs, ko + 4u * e);
        norm_rope16(kn, w->qk_norm + HD, trig, a.eps);
        if (slot == 0) {
            const Rs rk = rsrc(w->keys), rv = rsrc(w->values);
            const unsigned co = ((unsigned(pos) * NKV + unsigned(kvh)) * HD + sub * 16u) * 4u;
            const unsigned vo = SOFF(value) + (unsigned(kvh) * HD + sub * 16u) * 4u;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float vv = ldx(rs, vo + 4u * e);
                lw[sub * 16 + e] = kn[e];
                lw[HD + sub * 16 + e] = vv;
                stp(rk, co + 4u * e, kn[e]);
                stp(rv, co + 4u * e, vv);
            }
        }
        compiler_fence();
        patch_new(wb, lw, begin, pos);
    }
    const float scale = 1.f / 16.f;  // 1 / sqrt(256)
    int held = begin;  // wb holds the K/V chunk starting here (prefetched: the first)
#pragma unroll 1
    for (int g = 0; g < NH / NKV; ++g) {
        const int h = kvh * (NH / NKV) + g;
        float q[16];
        const unsigned qo = SOFF(mixed) + (unsigned(h) * 2u * HD + sub * 16u) * 4u;
#pragma unroll
        for (int e = 0; e < 16; ++e) q[e] = ldx(rs, qo + 4u * e);
        norm_rope16(q, w->qk_norm, trig, a.eps);
        float m = -INFINITY, lsum = 0.f, acc[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll 1
        for (int first = begin; first < end; first += SPAN) {
            if (first != held) {  // spans longer than one chunk (contexts over SPAN * SMAX)
                load_kv_chunk(w, kvh, first, pos, wb);
                if (has_new) patch_new(wb, lw, first, pos);
                held = first;
            }
#pragma unroll
            for (int step = 0; step < SPAN / 4; ++step) {
                const int pp = first + 4 * step + int(slot);
                float sc = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const f4 kv4 = wb[step * 8 + e];
                    sc = fmaf(q[4 * e], kv4.x, sc);
                    sc = fmaf(q[4 * e + 1], kv4.y, sc);
                    sc = fmaf(q[4 * e + 2], kv4.z, sc);
                    sc = fmaf(q[4 * e + 3], kv4.w, sc);
                }
                sc = group_sum<16>(sc) * scale;
                if (pp < end) {
                    const float mn = fmaxf(m, sc);
                    const float corr = expf(m - mn);
                    const float pw = expf(sc - mn);
                    lsum = lsum * corr + pw;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const f4 vv4 = wb[step * 8 + 4 + e];
                        acc[4 * e] = acc[4 * e] * corr + pw * vv4.x;
                        acc[4 * e + 1] = acc[4 * e + 1] * corr + pw * vv4.y;
                        acc[4 * e + 2] = acc[4 * e + 2] * corr + pw * vv4.z;
                        acc[4 * e + 3] = acc[4 * e + 3] * corr + pw * vv4.w;
                    }
                    m = mn;
                }
            }
        }
        // merge the 4 position slots
#pragma unroll
        for (int o = 16; o < 64; o <<= 1) {
            const float mo = __shfl_xor(m, o, 64), lo = __shfl_xor(lsum, o, 64);
            const float mn = fmaxf(m, mo);
            const float c0 = m == -INFINITY ? 0.f : expf(m - mn), c1 = mo == -INFINITY ? 0.f : expf(mo - mn);
            lsum = lsum * c0 + lo * c1;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[e] = acc[e] * c0 + __shfl_xor(acc[e], o, 64) * c1;
            m = mn;
        }
        const unsigned slotix = unsigned(h) * SMAX + unsigned(sp);
        if (lane == 0) {
            stx(rs, SOFF(pml) + slotix * 8u, m);
            stx(rs, SOFF(pml) + slotix * 8u + 4u, lsum);
        }
        if (slot == 0) {
            const unsigned ao = SOFF(pacc) + (slotix * HD + sub * 16u) * 4u;
#pragma unroll
            for (int e = 0; e < 16; ++e) stx(rs, ao + 4u * e, acc[e]);
        }
    }
}

// ---- T_COMB: merge the splits (log-sum-exp) and apply the sigmoid gate
// (reference.h:171-200); one wave per (head, 4 dims), lanes over splits.
constexpr int COMB_PER_LANE = SMAX / 64;
__device__ void phase_comb(const Args& a, Rs rs, int u) {
    if (u >= COMB_WAVES) return;
    const unsigned lane = lane_id();
    const int len = a.pos + 1, span = attn_span(len), splits = (len + span - 1) / span;
    const int h = u / (HD / 4), c4 = u % (HD / 4);
    float mv[COMB_PER_LANE];
    float mm = -INFINITY;
#pragma unroll
    for (int k = 0; k < COMB_PER_LANE; ++k) {
        const int s = int(lane) + 64 * k;
        mv[k] = s < splits ? ldx(rs, SOFF(pml) + (unsigned(h) * SMAX + unsigned(s)) * 8u) : -INFINITY;
        mm = fmaxf(mm, mv[k]);
    }
    mm = wave_max(mm);
    float den = 0.f;
    f4 num = f4(0.f);
#pragma unroll
    for (int k = 0; k < COMB_PER_LANE; ++k) {
        const int s = int(lane) + 64 * k;
        if (s < splits) {
            const unsigned ix = unsigned(h) * SMAX + unsigned(s);
            const float wgt = expf(mv[k] - mm);
            den += ldx(rs, SOFF(pml) + ix * 8u + 4u) * wgt;
            num += ldx4(rs, SOFF(pacc) + (ix * HD + unsigned(4 * c4)) * 4u) * wgt;
        }
    }
    den = wave_sum(den);
    num.x = wave_sum(num.x);
    num.y = wave_sum(num.y);
    num.z = wave_sum(num.z);
    num.w = wave_sum(num.w);
    if (lane < 4) {
        const float val = lane == 0 ? num.x : lane == 1 ? num.y : lane == 2 ? num.z : num.w;
        const int d = 4 * c4 + int(lane);
        const float gate = ldx(rs, SOFF(mixed) + unsigned(h * 2 * HD + HD + d) * 4u);
        stx(rs, SOFF(ctx) + unsigned(h * HD + d) * 4u, (val / den) * sigmoidf_(gate));
    }
}

// ---- T_O: after = x + o . ctx
__device__ void phase_o(const Args& a, Rs rs, int L, int u, const f4* wb) {
    if (u >= H) return;
    const unsigned lo = 16u * lane_id();
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < NH * HD / 256; ++v) acc = fdot4(wb[v], ldx4(rs, SOFF(ctx) + lo + 1024u * v), acc);
    acc = wave_sum(acc);
    if (lane_id() == 0) stx(rs, SOFF(after) + 4u * unsigned(u), input_at(a, rs, L, u) + acc);
}

// ---- T_LM: logits = lm_head . final RMSNorm(x); each wave streams its rows 4
// at a time with the next 4 in flight; per-wave (max, first index,
// non-finite count).
constexpr int LM_G = 4;
__device__ __forceinline__ int lm_rows_per_wave(int vocab) { return (vocab + NW - 1) / NW; }
__device__ __forceinline__ void lm_load(Rs lm, int row0, int row_end, f4* buf) {
#pragma unroll
    for (int r = 0; r < LM_G; ++r)
        if (row0 + r < row_end) {
            const unsigned lo = 16u * lane_id(), ro = unsigned(row0 + r) * unsigned(H * 4);
#pragma unroll
            for (int v = 0; v < 4; ++v) buf[r * 4 + v] = ldw(lm, lo + 1024u * v, ro);
        }
}
__device__ __forceinline__ void lm_rows(Rs lg, const f4* buf, const f4 (&xv)[4], int row0, int row_end, float& best,
                                        unsigned& at, unsigned& bad) {
#pragma unroll
    for (int r = 0; r < LM_G; ++r) {
        const int row = row0 + r;
        if (row < row_end) {
            float acc = 0.f;
#pragma unroll
            for (int v = 0; v < 4; ++v) acc = fdot4(buf[r * 4 + v], xv[v], acc);
            acc = wave_sum(acc);
            if (lane_id() == 0) stp(lg, 4u * unsigned(row), acc);
            if (!isfinite(acc)) {
                ++bad;
            } else if (acc > best) {
                best = acc;
                at = unsigned(row);
            }
        }
    }
}
__device__ __forceinline__ void prefetch_lm(const Args& a, int u, f4* wb) {
    const int rpw = lm_rows_per_wave(a.vocab), row0 = u * rpw, row_end = min(a.vocab, row0 + rpw);
    lm_load(rsrc(a.lm_head), row0, row_end, wb);
}
__device__ void phase_lm(const Args& a, Rs rs, int u, f4* wb) {
    f4 xv[4];
    const unsigned lo = 16u * lane_id();
#pragma unroll
    for (int v = 0; v < 4; ++v) xv[v] = ldx4(rs, SOFF(x) + lo + 1024u * v);
    norm_chunks(xv, a.final_norm, a.eps);
    const int rpw = lm_rows_per_wave(a.vocab), row0 = u * rpw, row_end = min(a.vocab, row0 + rpw);
    const Rs lm = rsrc(a.lm_head), lg = rsrc(a.logits);
    float best = -INFINITY;
    unsigned at = 0xffffffffu, bad = 0;
    f4 nb[4 * LM_G];
    for (int r = row0; r < row_end; r += 2 * LM_G) {
        lm_load(lm, r + LM_G, row_end, nb);
        lm_rows(lg, wb, xv, r, row_end, best, at, bad);
        if (r + LM_G >= row_end) break;
        lm_load(lm, r + 2 * LM_G, row_end, wb);
        lm_rows(lg, nb, xv, r + LM_G, row_end, best, at, bad);
    }
    if (lane_id() == 0) {
        const unsigned o = SOFF(lmpart) + unsigned(u) * 12u;
        stx(rs, o, best);
        stx(rs, o + 4, __uint_as_float(at));
        stx(rs, o + 8, __uint_as_float(bad));
    }
}

// ---- T_ARG: merge the per-wave maxima (first index of the maximum, non-finite
// count; reference.h:222-230).
__device__ void phase_arg(const Args& a, Rs rs) {
    const unsigned lane = lane_id();
    float best = -INFINITY;
    unsigned at = 0xffffffffu, bad = 0;
    for (int i = int(lane); i < NW; i += 64) {
        const unsigned o = SOFF(lmpart) + unsigned(i) * 12u;
        const float v = ldx(rs, o);
        const unsigned idx = __float_as_uint(ldx(rs, o + 4));
        bad += __float_as_uint(ldx(rs, o + 8));
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
        const Rs pk = rsrc(a.picks);
        stp(pk, 0, float(at));
        stp(pk, 4, float(bad));
    }
}

// ---------------------------------------------------------------- the kernel
__device__ __forceinline__ void prefetch(const Args& a, int q, int u, f4* wb) {
    if (q >= a.nphases) return;
    const LayerP w = layer(a, player(a, q));
    switch (ptype(a, q)) {
    case T_DIN: prefetch_din(w, u, wb); break;
    case T_MIX: prefetch_mix(w, u, wb); break;
    case T_DOUT: prefetch_row<VD>(w->out, u, H, wb); break;
    case T_GLU: prefetch_glu(w, u, wb); break;
    case T_DOWN: prefetch_row<I>(w->down, u, H, wb); break;
    case T_AQKV: prefetch_aqkv(w, u, wb); break;
    case T_ATTN: prefetch_attn(w, u, a.pos, wb); break;
    case T_O: prefetch_row<NH * HD>(w->o, u, H, wb); break;
    case T_LM: prefetch_lm(a, u, wb); break;
    default: break;
    }
}

__global__ __launch_bounds__(THREADS, 1) void decode_kernel(Args a) {
    __shared__ Lds l;
    // wave-uniform (readfirstlane lets the compiler keep indices and buffer
    // descriptors derived from it in SGPRs)
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int unit = wave * BLOCKS + int(blockIdx.x);  // rows spread wave-major over blocks
    if (threadIdx.x == 0) {
        for (int i = 0; i < 4; ++i) l.done[i] = 0;
        l.seen = 0;
        l.fail = 0;
    }
    __syncthreads();
    const bool poller = wave == 0;
    const Rs rs = rsrc(a.s);
    f4 wb[WBUF];
    prefetch(a, 0, unit, wb);
    for (int p = 0; p < a.nphases; ++p) {
        const int t = ptype(a, p);
        if (t == T_ARG) {
            if (blockIdx.x == 0 && wave == 0 && wait_phase(a, l, p - 1, true)) phase_arg(a, rs);
            return;
        }
        if (p > 0 && !wait_phase(a, l, p - 1, poller)) return;
        const int L = player(a, p);
        const LayerP w = layer(a, L);
        const int u = opaque_uniform(unit);
        switch (t) {
        case T_DIN: phase_din(a, rs, w, L, u, wb); break;
        case T_MIX: phase_mix(a, rs, w, L, u, wb, l); break;
        case T_DOUT: phase_dout(a, rs, w, L, u, wb); break;
        case T_GLU: phase_glu(a, rs, w, u, wb); break;
        case T_DOWN: phase_down(rs, u, wb); break;
        case T_AQKV: phase_aqkv(a, rs, w, L, u, wb); break;
        case T_ATTN: phase_attn(a, rs, w, u, wb, l); break;
        case T_COMB: phase_comb(a, rs, u); break;
        case T_O: phase_o(a, rs, L, u, wb); break;
        case T_LM: phase_lm(a, rs, u, wb); break;
        default: break;
        }
        signal(a, l, p);
        prefetch(a, p + 1, opaque_uniform(unit), wb);
    }
}

}  // namespace dec
}  // namespace qr

// ---------------------------------------------------------------- plan (host)
struct QrDecodePlan {
    qr::dec::Args args;
    QrDecodeLayer* layers = nullptr;
    qr::dec::Scratch* scratch = nullptr;
    qr::dec::Sync* sync = nullptr;
    float* denom = nullptr;
    int capacity = 0;
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
    // every buffer offset is 32-bit: the largest matrix and cache must stay under 4 GiB
    if (double(d.vocab) * H * 4.0 >= 4294967296.0 || double(d.capacity) * NKV * HD * 4.0 >= 4294967296.0)
        return "one-launch decode: vocabulary or capacity beyond 32-bit offsets";
    if (!d.embedding || !d.final_norm || !d.logits || !d.picks || !d.layer)
        return "one-launch decode: missing buffer";
    int phases = 2;
    for (int l = 0; l < d.layers; ++l) phases += d.layer[l].attention ? 6 : 5;
    if (phases > MAXPH || phases >= 1023) return "one-launch decode: too many phases";
    return nullptr;
}

int decode_plan_create(const QrDecodeDesc& d, QrDecodePlan** out, hipStream_t s, const char** why) {
    using namespace dec;
    *out = nullptr;
    if ((*why = decode_unsupported(d))) return -1;
    int dev = 0, cus = 0, per_cu = 0, coop = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    (void)hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev);
    if (!coop || hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_kernel, THREADS, 0) != hipSuccess ||
        per_cu * cus < BLOCKS) {
        *why = "one-launch decode: 256 co-resident blocks do not fit this device";
        return -1;
    }
    auto* p = new QrDecodePlan;
    std::memset(&p->args, 0, sizeof(p->args));
    p->capacity = d.capacity;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&p->layers), sizeof(QrDecodeLayer) * size_t(d.layers));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&p->scratch), sizeof(Scratch));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&p->sync), sizeof(Sync));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&p->denom), sizeof(float) * ROT / 2);
    // RoPE denominators theta^(2i / rot) by the host libm (the reference's
    // expression, src/attention.rs:49-50), as the op path's table
    std::vector<float> denom(ROT / 2);
    for (int i = 0; i < ROT / 2; ++i) denom[size_t(i)] = powf(d.theta, float(2 * i) / float(ROT));
    if (e == hipSuccess)
        e = hipMemcpyAsync(p->layers, d.layer, sizeof(QrDecodeLayer) * size_t(d.layers), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(p->denom, denom.data(), sizeof(float) * ROT / 2, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemsetAsync(p->sync, 0, sizeof(Sync), s);
    if (e == hipSuccess) e = hipMemsetAsync(p->scratch, 0, sizeof(Scratch), s);
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
    a.rope_denom = p->denom;
    a.s = p->scratch;
    a.sync = p->sync;
    a.vocab = d.vocab;
    a.eps = d.eps;
    a.epoch = 0;
    static const uint8_t delta[5] = {T_DIN, T_MIX, T_DOUT, T_GLU, T_DOWN};
    static const uint8_t attn[6] = {T_AQKV, T_ATTN, T_COMB, T_O, T_GLU, T_DOWN};
    int n = 0;
    for (int l = 0; l < d.layers; ++l) {
        const uint8_t* seq = d.layer[l].attention ? attn : delta;
        const int cnt = d.layer[l].attention ? 6 : 5;
        for (int k = 0; k < cnt; ++k) a.phase[n++] = uint32_t(seq[k]) | uint32_t(l) << 8;
    }
    a.phase[n++] = T_LM;
    a.phase[n++] = T_ARG;
    a.nphases = n;
    *out = p;
    return 0;
}

void decode_plan_free(QrDecodePlan* p) {
    if (!p) return;
    if (p->layers) (void)hipFree(p->layers);
    if (p->scratch) (void)hipFree(p->scratch);
    if (p->sync) (void)hipFree(p->sync);
    if (p->denom) (void)hipFree(p->denom);
    delete p;
}

int decode_step(QrDecodePlan* p, int token, int position, hipStream_t s) {
    using namespace dec;
    Args& a = p->args;
    if (token < 0 || token >= a.vocab || position < 0 || position >= p->capacity) return int(hipErrorInvalidValue);
    a.token = token;
    a.pos = position;
    a.epoch = (a.epoch + 1) & 0x3fffffu;
    if (a.epoch == 0) a.epoch = 1;
    void* args[] = {&a};
    return int(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(decode_kernel), dim3(BLOCKS), dim3(THREADS),
                                          args, 0, s));
}

}  // namespace qr
