// stream.hip -- the persistent token kernel for gfx950 (see stream.h for the
// workgroup organisation).  One launch = one token of the decode loop
// (reference: infer/forward.odin:17-146 for the layer arithmetic,
// infer/metal.odin:443-514 for the f16 KV cache and its attention,
// sampler/sampler.odin:79-89 for the greedy pick).
//
// Stages of a launch, each ended by a grid barrier (except the last):
//   EMBED   argmax of the previous launch's partials -> token; this
//           workgroup's rows of x = token_embd[token]; quantized
//           attn_norm_0 * x and the partial sum of squares
//   per layer:
//   QKV     y = W{q,k,v} rmsnorm(x)        -> q, k, v (f32)
//   ATTN    q/k head norm + RoPE, K/V[pos] to the f16 cache, split-L
//           attention over 64-position chunks -> (o, m, l) partials
//   COMB    merge of the partials of 16 output dims per workgroup -> att
//   WO      x += Wo att                     -> quantized ffn_norm * x
//   GU      h = silu(Wg rmsnorm(x)) * (Wu rmsnorm(x))
//   DOWN    x += Wd h                       -> quantized next norm * x
//   VOCAB   logits = Wout rmsnorm(x), argmax partial per workgroup
//
// Inter-stage vectors are quantized by their producer (the workgroup that
// owns the rows) into the 22-bit three-plane form that the GEMV consumes
// (stream.h, qvec_bytes), with the RMSNorm weight of the consumer already
// multiplied in; the consumer applies the norm's scalar 1/sqrt(mean(x^2)+eps)
// to each output row.  Quantization is scale invariant, so this equals
// quantizing the normalized vector up to f32 rounding.

#include <math.h>

#include <algorithm>
#include <type_traits>

#include "device_common.h"
#include "stream.h"

namespace oi {

constexpr float XQ_MAX_S = 32767.0f;  // 2^15 - 1: 16-bit activations
constexpr int NTOT_IO = S_NCW + S_NLD;  // index of the I/O wave
// Pieces of the next weight stage the loaders may request before the compute
// waves start it.  Loads run ahead of a stage barrier only this far: the
// I/O wave's stores, barrier atomics and gathers queue behind loads in flight.
#ifndef OI_STREAM_LEAD
#define OI_STREAM_LEAD 4
#endif
constexpr uint32_t S_LEAD = OI_STREAM_LEAD;
constexpr uint64_t SPIN_TICKS = 200000000ull;  // 2 s of the 100 MHz real-time clock

#define LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

// ------------------------------------------------------------ coherence --
// Values exchanged between workgroups within a launch are written and read
// with device-scope (sc1) accesses: relaxed agent-scope atomics, which reach
// the point of coherence of all XCDs, so no cache writeback or invalidate is
// needed.  Ordering: a workgroup waits for its stores to complete
// (s_waitcnt vmcnt(0)) before it arrives at the barrier.
static __device__ __forceinline__ void st_f(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
static __device__ __forceinline__ void st_u(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
static __device__ __forceinline__ void st_i(int32_t *p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
static __device__ __forceinline__ float ld_f(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
static __device__ __forceinline__ uint64_t ld_u64(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
static __device__ __forceinline__ void vm_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

static __device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// Barrier of the compute waves and the I/O wave (the loader waves never
// wait for them, so s_barrier cannot be used): a counter in LDS.  Each
// wave's LDS writes are complete before it arrives (lgkmcnt(0)); LDS
// accesses are performed in order, so a wave that sees the count sees them.
static __device__ __forceinline__ void lds_bar(uint32_t *ctr, uint32_t &target) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    target += S_NCW + 1;
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) __builtin_amdgcn_s_sleep(1);
    asm volatile("" ::: "memory");
}
static __device__ __forceinline__ uint32_t lds_ld(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
static __device__ __forceinline__ void lds_st(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Read-only plan tables through the constant address space: with a uniform
// index these become scalar loads, which do not touch vmcnt (a vector load
// here would make the compiler wait for every direct-to-LDS load in flight).
#if defined(__HIP_DEVICE_COMPILE__)
#define CST(p) ((const __attribute__((address_space(4))) std::remove_cv_t<std::remove_pointer_t<decltype(p)>> *)(p))
#else
#define CST(p) (p)  // host pass of the same source: no address spaces
#endif

// debugging trace (StreamArgs::trace), lane 0: slots 0..7 of (stage,
// workgroup) are clock stamps (TRACE), 8 + w the ticks compute wave w spent
// waiting for its ring in the stage, 16 + 4 L .. of the last stage loader
// L's counts of pieces loaded, idle slots and sleeps (TRACE_SET)
#define TRACE_SET(a, stage, k, v)                                                                          \
    do {                                                                                                    \
        if ((a).trace && (threadIdx.x & 63) == 0)                                                           \
            (a).trace[((size_t)(stage) * (a).G + blockIdx.x) * S_TR_SLOTS + (k)] = (v);                     \
    } while (0)
#define TRACE(a, stage, k) TRACE_SET(a, stage, k, __builtin_amdgcn_s_memrealtime())

// ------------------------------------------------------------ LDS layout --
struct __attribute__((aligned(16))) Misc {
    uint32_t filled[S_NCW];    // pieces of each compute wave's stream written into its ring
    uint32_t consumed[S_NCW];  // stream bytes each compute wave has consumed
    uint32_t allow[S_NCW];     // pieces of each stream the loaders may request so far
    uint32_t bar;              // barrier counter of the compute and I/O waves
    float s_norm;            // RMSNorm scale of the current stage's input
    int32_t abort;
    int32_t token, pos;
    int32_t kv_store[2];     // per attention half: 1 if it holds K/V[pos] to store
    float red[16];
    int32_t redi[16];
    float xres[256];         // this workgroup's rows of the residual stream x
    float nrm[256];          // the next norm weights of those rows (requested a stage ahead)
    float yo_pad[4];
    uint8_t qstage[16 * 32]; // producer quantization staging (16 chunks)
};

struct Lds {
    uint8_t *ring;   // S_NCW * S_RING_BYTES
    uint8_t *xr;     // stage input vector (quantized) / attention scratch
    Misc *misc;
    float *yo;       // this workgroup's stage outputs
};

static __device__ __forceinline__ int cslot(int C) { return (C & ~3) | ((C & 3) ^ ((C >> 4) & 3)); }

// ----------------------------------------------------- weight stream ring --
// Compute wave's view of its ring: piece p of its stream (1 KB) sits at
// ring slot p % S_RING once filled >= p + 1; the wave publishes the stream
// bytes it has consumed so the loader can reuse their slots.
struct Ring {
    uint32_t consumed;   // stream bytes consumed
    uint8_t *lds;        // the compute wave's ring
    const uint32_t *filled;
    uint32_t *consumed_p;
    uint32_t *allow_p;   // loader limit of this stream (pieces)
    uint32_t *abort_p;   // the workgroup's abort flag (LDS)
    int32_t *err_p;      // the launch's error word (state)
    bool trace;          // debugging: count the ticks spent waiting
    uint64_t wait_ticks;
};

// compute wave: bytes [.., end) of its stream are in its ring once this returns
// (on an abort, or after SPIN_TICKS without progress, which aborts the
// launch: the stage then completes on stale ring data and the host reports
// the error)
static __device__ __forceinline__ void ring_wait(Ring &r, uint32_t end) {
    const uint32_t need = uni((end + 1023) / 1024);
    if (lds_ld(r.filled) < need) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (lds_ld(r.filled) < need && !lds_ld(r.abort_p)) {
            if (__builtin_amdgcn_s_memrealtime() - t0 > SPIN_TICKS) {
                if ((threadIdx.x & 63) == 0) {
                    lds_st(r.abort_p, 1u);
                    __hip_atomic_store(r.err_p, (int32_t)S_ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (r.trace) r.wait_ticks += __builtin_amdgcn_s_memrealtime() - t0;
    }
    asm volatile("" ::: "memory");
}
// compute wave: stream bytes before `off` are consumed (their ring slots may be refilled)
static __device__ __forceinline__ void ring_release(Ring &r, uint32_t off) {
    asm volatile("" ::: "memory");  // the ring reads are issued first (LDS performs a wave's accesses in order)
    r.consumed = off;
    if ((threadIdx.x & 63) == 0) lds_st(r.consumed_p, off);
}

// 16-byte read at stream offset `base + off` (off < S_RING_BYTES)
static __device__ __forceinline__ const uint8_t *rp(const Ring &r, uint32_t bmod, uint32_t off) {
    uint32_t o = bmod + off;
    if (o >= (uint32_t)S_RING_BYTES) o -= S_RING_BYTES;
    return r.lds + o;
}

// ---------------------------------------------------------------- GEMV --
static __device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
static __device__ __forceinline__ uint32_t udot4(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_udot4(a, b, c, false);
}
// first product of a chain: the three-operand form with an inline zero
// (the compiler would otherwise zero a register for the accumulate form)
static __device__ __forceinline__ int sdot4z(uint32_t a, uint32_t b) {
    int d;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
// sum of w * q over a chunk part from the hi (signed) and lo (unsigned) planes
static __device__ __forceinline__ float psum(int h, uint32_t l) { return (float)((h << 8) + (int)l); }

// x slice of one lane: 4 chunks of 16 elements
struct XS {
    u32x4 h[4], l[4];
    float xs[4], s[4];
};
static __device__ __forceinline__ void x_load(const uint8_t *xr, int K, const int (&C)[4], XS &x) {
    const int nch = K / 16;
    const u32x4 *hi = (const u32x4 *)xr, *lo = hi + nch;
    const float *xs = (const float *)(lo + nch), *s16 = xs + nch;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        x.h[c] = hi[cslot(C[c])];
        x.l[c] = lo[cslot(C[c])];
        x.xs[c] = xs[C[c]];
        x.s[c] = s16[C[c]];
    }
}
// chunks of unit u: Q4_K / Q8_0 4u..4u+3; Q6_K the four 16-element runs
// 128h + 32k + l0 of its super-block half (ggml/quant.odin:212-247)
template <int T>
static __device__ __forceinline__ void unit_chunks(int u, int (&C)[4]) {
#pragma unroll
    for (int k = 0; k < 4; k++)
        C[k] = T == T_Q6_K ? 16 * (u >> 2) + 8 * ((u >> 1) & 1) + (u & 1) + 2 * k : 4 * u + k;
}

// Q4_K: lane's unit = group pair p = l & 3 of super-block; chunks 0,1 low
// nibbles (group 2p), 2,3 high nibbles (group 2p+1)
template <class RD>
static __device__ __forceinline__ float dot_q4k(const RD &rp, int lane, const XS &x) {
    const u32x4 q0 = *(const u32x4 *)rp(16 * lane);
    const u32x4 q1 = *(const u32x4 *)rp(1024 + 16 * lane);
    const u32x4 hd = *(const u32x4 *)rp(2048 + 16 * (lane >> 2));
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    int ah[4];
    uint32_t al[4];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t lo = qw[k] & 0x0F0F0F0Fu, hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
        const int c0 = k >> 2, c1 = 2 + (k >> 2), e = k & 3;
        if (e == 0) {
            ah[c0] = sdot4z(lo, x.h[c0][e]);
            ah[c1] = sdot4z(hi, x.h[c1][e]);
            al[c0] = udot4(lo, x.l[c0][e], 0u);
            al[c1] = udot4(hi, x.l[c1][e], 0u);
        } else {
            ah[c0] = sdot4(lo, x.h[c0][e], ah[c0]);
            ah[c1] = sdot4(hi, x.h[c1][e], ah[c1]);
            al[c0] = udot4(lo, x.l[c0][e], al[c0]);
            al[c1] = udot4(hi, x.l[c1][e], al[c1]);
        }
    }
    const float d = h2f(hd.x & 0xFFFFu), dmin = h2f(hd.x >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(lane & 3, hd.y, hd.z, hd.w, sc0, m0, sc1, m1);
    const float dA = psum(ah[0], al[0]) * x.xs[0] + psum(ah[1], al[1]) * x.xs[1];
    const float dB = psum(ah[2], al[2]) * x.xs[2] + psum(ah[3], al[3]) * x.xs[3];
    return d * ((float)sc0 * dA + (float)sc1 * dB) - dmin * ((float)m0 * (x.s[0] + x.s[1]) + (float)m1 * (x.s[2] + x.s[3]));
}

template <class RD>
static __device__ __forceinline__ float dot_q6k(const RD &rp, int lane, const XS &x) {
    const u32x4 a0 = *(const u32x4 *)rp(16 * lane);
    const u32x4 a1 = *(const u32x4 *)rp(1024 + 16 * lane);
    const u32x4 qv = *(const u32x4 *)rp(2048 + 16 * lane);
    const u32x2 scw = *(const u32x2 *)rp(3072 + 16 * (lane >> 2) + 8 * ((lane >> 1) & 1));
    const uint32_t dd = *(const uint16_t *)rp(3328 + 2 * (lane >> 2));
    const uint32_t l0[4] = {a0.x, a0.y, a0.z, a0.w}, l1[4] = {a1.x, a1.y, a1.z, a1.w};
    const uint32_t qh[4] = {qv.x, qv.y, qv.z, qv.w};
    int ah[4];
    uint32_t al[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // 6-bit values v = q + 32 (0..63) of the four 16-element runs, 4 per word
        const uint32_t v[4] = {(l0[i] & 0x0F0F0F0Fu) | ((qh[i] & 0x03030303u) << 4),
                               (l1[i] & 0x0F0F0F0Fu) | (((qh[i] >> 2) & 0x03030303u) << 4),
                               ((l0[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> 4) & 0x03030303u) << 4),
                               ((l1[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> 6) & 0x03030303u) << 4)};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (i == 0) {
                ah[k] = sdot4z(v[k], x.h[k][i]);
                al[k] = udot4(v[k], x.l[k][i], 0u);
            } else {
                ah[k] = sdot4(v[k], x.h[k][i], ah[k]);
                al[k] = udot4(v[k], x.l[k][i], al[k]);
            }
        }
    }
    const uint32_t sw[2] = {scw.x, scw.y};
    const int bsh = lane & 1;
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int bi = bsh + 2 * k;
        const float s = (float)(int8_t)((sw[bi >> 2] >> ((bi & 3) * 8)) & 0xFFu);
        acc += s * (psum(ah[k], al[k]) * x.xs[k] - 32.f * x.s[k]);
    }
    return h2f(dd) * acc;
}

// Q8_0: signed weights against the unsigned lo plane as (w + 128) . lo - 128 sum(lo)
template <class RD>
static __device__ __forceinline__ float dot_q80(const RD &rp, int lane, const XS &x) {
    int ah[4];
    uint32_t al[4], ls[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const u32x4 w = *(const u32x4 *)rp(1024 * c + 16 * lane);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t wu = w[e] ^ 0x80808080u;
            if (e == 0) {
                ah[c] = sdot4z(w[e], x.h[c][e]);
                al[c] = udot4(wu, x.l[c][e], 0u);
                ls[c] = udot4(0x01010101u, x.l[c][e], 0u);
            } else {
                ah[c] = sdot4(w[e], x.h[c][e], ah[c]);
                al[c] = udot4(wu, x.l[c][e], al[c]);
                ls[c] = udot4(0x01010101u, x.l[c][e], ls[c]);
            }
        }
    }
    const uint32_t dw = *(const uint32_t *)rp(4096 + 4 * lane);
    float p[4];
#pragma unroll
    for (int c = 0; c < 4; c++) p[c] = (float)((ah[c] << 8) + (int)al[c] - 128 * (int)ls[c]);
    return h2f(dw & 0xFFFFu) * (p[0] * x.xs[0] + p[1] * x.xs[1]) + h2f(dw >> 16) * (p[2] * x.xs[2] + p[3] * x.xs[3]);
}

template <int T, class RD>
static __device__ __forceinline__ float dot_t(const RD &rp, int lane, const XS &x) {
    if (T == T_Q4_K) return dot_q4k(rp, lane, x);
    if (T == T_Q6_K) return dot_q6k(rp, lane, x);
    return dot_q80(rp, lane, x);
}

// Reads of a step at ring offset bm: contiguous when the step does not
// cross the ring end (one address add, then immediate offsets), wrapped
// per read otherwise.
struct RdLin {
    const uint8_t *p;
    __device__ __forceinline__ const uint8_t *operator()(uint32_t off) const { return p + off; }
};
struct RdWrap {
    const uint8_t *lds;
    uint32_t bm;
    __device__ __forceinline__ const uint8_t *operator()(uint32_t off) const {
        uint32_t o = bm + off;
        if (o >= (uint32_t)S_RING_BYTES) o -= S_RING_BYTES;
        return lds + o;
    }
};

// One run of rows [row0, row0+nrows) of one segment: steps of NR = 64/lpr
// rows x lpr units; `soff` is the stream offset of the run's first step.
// Row results (times `scale`; SwiGLU for pairs) go to yo[vrow - v0].
template <int T, bool PAIR>
static __device__ void gemv_run(const StreamArgs &a, int cw, Ring &r, uint32_t &soff, const SKind &kd, const SRun &run,
                                const uint8_t *xr, float *yo, int v0, float scale, int tst) {
    const int lane = threadIdx.x & 63;
    const int lpr = (int)uni((uint32_t)kd.lpr), K = (int)uni((uint32_t)kd.K);
    const int nb = (K >> 6) / lpr, NR = 64 / lpr;
    const int j = lane & (lpr - 1), rsub = lane / lpr;
    constexpr uint32_t SB1 = (uint32_t)step_bytes(T), SB = SB1 * (PAIR ? 2 : 1);
    const int nrows = (int)uni((uint32_t)run.nrows);
    const int nrs = (nrows + NR - 1) / NR;
    XS x;
    int C[4];
    if (nb == 1) {
        unit_chunks<T>(j, C);
        x_load(xr, K, C, x);
    }
    if (tst >= 0 && cw % S_NCW == 0) TRACE(a, tst, 7);
    for (int rs = 0; rs < nrs; rs++) {
        float acc0 = 0.f, acc1 = 0.f;
        for (int b = 0; b < nb; b++) {
            if (nb > 1) {
                unit_chunks<T>(b * lpr + j, C);
                x_load(xr, K, C, x);
            }
            ring_wait(r, soff + SB);
            const uint32_t bm = uni(soff % (uint32_t)S_RING_BYTES);
            if (bm + SB <= (uint32_t)S_RING_BYTES) {
                const RdLin rd{r.lds + bm};
                acc0 += dot_t<T>(rd, lane, x);
                if (PAIR) acc1 += dot_t<T>(RdLin{r.lds + bm + SB1}, lane, x);
            } else {
                acc0 += dot_t<T>(RdWrap{r.lds, bm}, lane, x);
                if (PAIR) {
                    uint32_t bm1 = bm + SB1;
                    if (bm1 >= (uint32_t)S_RING_BYTES) bm1 -= S_RING_BYTES;
                    acc1 += dot_t<T>(RdWrap{r.lds, bm1}, lane, x);
                }
            }
            soff += SB;
            ring_release(r, soff);  // per step: a row step of nb steps may exceed the ring
        }
        acc0 = lane_group_sum(acc0, lpr);
        if (PAIR) acc1 = lane_group_sum(acc1, lpr);
        const int rr = rs * NR + rsub;
        if (j == 0 && rr < nrows) {
            float v = acc0 * scale;
            if (PAIR) {  // infer/forward.odin:128-133
#pragma clang fp contract(off)
                v *= 1.0f / (1.0f + expf(-v));
                v *= acc1 * scale;
            }
            yo[run.vrow + rr - v0] = v;
        }
    }
}

// All runs of compute wave cw in stage kind `kind`; soff advances to the
// next segment start (whole pieces).
static __device__ void gemv_stage(const StreamArgs &a, int cw, Ring &r, uint32_t &soff, int pl, const uint8_t *xr,
                                  float *yo, float scale, int tst) {
    pl = (int)uni((uint32_t)pl);
    const SKind kd = CST(a.kinds)[pl];
    const auto *wv = &CST(a.waves)[(size_t)pl * a.G * S_NCW + cw];
    const int v0 = CST(a.wgrows)[(size_t)pl * a.G + blockIdx.x].v0;
    const uint32_t start = soff;
    const int nruns = wv->nruns, npieces = wv->npieces;
    if ((threadIdx.x & 63) == 0) lds_st(r.allow_p, start / 1024 + (uint32_t)npieces + S_LEAD);
    for (int i = 0; i < nruns; i++) {
        const SRun run = wv->run[i];
        const int type = kd.seg[run.seg].type;
        if (i == 0 && cw % S_NCW == 0 && type >= 0) TRACE(a, tst, 3);
        if (kd.pair) {
            if (type == T_Q4_K) gemv_run<T_Q4_K, true>(a, cw, r, soff, kd, run, xr, yo, v0, scale, i == 0 ? tst : -1);
            else if (type == T_Q6_K) gemv_run<T_Q6_K, true>(a, cw, r, soff, kd, run, xr, yo, v0, scale, i == 0 ? tst : -1);
            else gemv_run<T_Q8_0, true>(a, cw, r, soff, kd, run, xr, yo, v0, scale, i == 0 ? tst : -1);
        } else if (type == T_Q4_K) {
            gemv_run<T_Q4_K, false>(a, cw, r, soff, kd, run, xr, yo, v0, scale, i == 0 ? tst : -1);
        } else if (type == T_Q6_K) {
            gemv_run<T_Q6_K, false>(a, cw, r, soff, kd, run, xr, yo, v0, scale, i == 0 ? tst : -1);
        } else {
            gemv_run<T_Q8_0, false>(a, cw, r, soff, kd, run, xr, yo, v0, scale, i == 0 ? tst : -1);
        }
    }
    soff = start + (uint32_t)npieces * 1024u;
    ring_release(r, soff);
}

// Grid barrier over cumulative counters: workgroup w adds 1 to counter
// w % S_NC when it finishes a stage (grid_arrive, after its stores have
// completed); barrier b of launch `seq` is passed once every counter holds
// (seq * nb + b + 1) times the number of workgroups mapped to it.  A
// workgroup cannot arrive at barrier b+1 before barrier b is passed, so the
// counts cannot run ahead.
static __device__ __forceinline__ void grid_arrive(const StreamArgs &a) {
    if ((threadIdx.x & 63) == 0)
        __hip_atomic_fetch_add(a.bar + (size_t)(blockIdx.x % S_NC) * 32, (uint64_t)1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}
// false on timeout (SPIN_TICKS)
static __device__ bool grid_wait(const StreamArgs &a, uint64_t seq, int nb, int b) {
    const int lane = threadIdx.x & 63;
    const int per = a.G / S_NC + (lane < a.G % S_NC ? 1 : 0);  // workgroups on counter `lane`
    const uint64_t want = (seq * (uint64_t)nb + (uint64_t)b + 1) * (uint64_t)per;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (true) {
        bool ok = true;
        if (lane < S_NC) ok = ld_u64(a.bar + (size_t)lane * 32) >= want;
        if (__all(ok)) return true;
        if (__builtin_amdgcn_s_memrealtime() - t0 > SPIN_TICKS) return false;
        __builtin_amdgcn_s_sleep(2);
    }
}

// load `bytes` (multiple of 16) from a vector written in this launch into LDS
// with device-scope direct-to-LDS loads (1 KB per instruction)
static __device__ __forceinline__ void io_dma(const uint8_t *src, uint8_t *dst, int bytes) {
    const int lane = threadIdx.x & 63;
    for (int off = 0; off < bytes; off += 1024)
        if (off + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds((const void *)(src + off + lane * 16), LDS_PTR(dst + off), 16, 0,
                                             16 /* sc1 */);
}

// 512 bytes (lanes 0..31); aux 16: device-scope (written in this launch), 0: read-only data
static __device__ __forceinline__ void io_dma_half(const uint8_t *src, uint8_t *dst, int aux) {
    const int lane = threadIdx.x & 63;
    if (lane < 32) {
        if (aux) __builtin_amdgcn_global_load_lds((const void *)(src + lane * 16), LDS_PTR(dst), 16, 0, 16);
        else __builtin_amdgcn_global_load_lds((const void *)(src + lane * 16), LDS_PTR(dst), 16, 0, 0);
    }
}

// RMSNorm scale from the partial sums of squares (ops.odin:7-19 computes
// 1/sqrt(sum(x^2)/n + eps))
static __device__ float io_norm_scale(const StreamArgs &a) {
    const int lane = threadIdx.x & 63;
    float s = 0.f;
    for (int i = lane; i < a.G; i += 64) s += ld_f(a.ssq + i);
    s = wave_sum(s);
    return 1.0f / sqrtf(s / (float)a.D + a.eps);
}

// Quantize n values (n a multiple of 16, <= 256) vals[i] * (w ? w[i] : 1)
// starting at element e0 (a multiple of 16) of a K-vector into the qvec at
// dst (device-scope stores).  Returns the sum of squares of vals (not
// weighted) in every lane.
static __device__ float io_quantize(const float *vals, const float *w, int n, int e0, int K, uint8_t *dst,
                                    uint8_t *stage) {
    const int lane = threadIdx.x & 63;
    const int nch = K / 16;
    float ssq = 0.f;
    for (int b = 0; b < n; b += 64) {
        const int i = b + lane;
        const bool ok = i < n;
        const float x = ok ? vals[i] : 0.f;
        ssq += x * x;
        float v = x;
        if (w && ok) {
#pragma clang fp contract(off)
            v = w[i] * x;
        }
        float amax = fabsf(v);
        amax = fmaxf(amax, OI_DPP(amax, 0xB1));
        amax = fmaxf(amax, OI_DPP(amax, 0x4E));
        amax = fmaxf(amax, OI_DPP(amax, 0x141));
        amax = fmaxf(amax, OI_DPP(amax, 0x140));  // max over the 16 lanes of the chunk
        const float sum = lane_group_sum(v, 16);
        const float inv = amax > 0.f ? XQ_MAX_S / amax : 0.f;
        const int q = (int)rintf(v * inv);
        const int cc = lane >> 4, k = lane & 15;  // chunk of this pass, element within the chunk
        stage[cc * 32 + k] = (uint8_t)((q >> 8) & 0xFF);
        stage[cc * 32 + 16 + k] = (uint8_t)(q & 0xFF);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // one wave: LDS accesses complete in order
        const int nc = min(4, (n - b) / 16);
        if (lane < nc * 8) {  // 8 words (2 planes x 16 bytes) per chunk
            const int c2 = lane / 8, pl = (lane % 8) / 4, wd = lane & 3;
            const int C = (e0 + b) / 16 + c2;
            const uint32_t word = *(const uint32_t *)(stage + c2 * 32 + pl * 16 + wd * 4);
            st_u((uint32_t *)(dst + (size_t)pl * nch * 16 + (size_t)cslot(C) * 16 + wd * 4), word);
        }
        if (ok && k == 0) {
            const int C = (e0 + i) / 16;
            st_f((float *)(dst + (size_t)nch * 32) + C, amax / XQ_MAX_S);
            st_f((float *)(dst + (size_t)nch * 36) + C, sum);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    return wave_sum(ssq);
}

static __device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// argmax candidates: (value, lowest index), first maximum wins
static __device__ __forceinline__ void wave_best(float &bv, int &bi) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, WAVE);
        const int oi = __shfl_xor(bi, o, WAVE);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
}

// bit-exact element of a dequantized row (ggml/quant.odin:76-247) in the
// GEMV plane layout (oi_kernels.h DMat)
static __device__ float emb_elem(const DMat &m, int row, int col) {
#pragma clang fp contract(off)
    switch (m.type) {
    case T_Q4_K: {
        const int sb = col >> 8, g = (col >> 5) & 7, l = col & 31, p = g >> 1;
        const size_t ui = (size_t)row * (m.cols >> 6) + 4 * sb + p;
        const uint8_t *hd = m.s + ((size_t)row * (m.cols >> 8) + sb) * 16;
        const uint32_t hw0 = *(const uint32_t *)hd, hw1 = *(const uint32_t *)(hd + 4),
                       hw2 = *(const uint32_t *)(hd + 8), hw3 = *(const uint32_t *)(hd + 12);
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(p, hw1, hw2, hw3, sc0, m0, sc1, m1);
        const float d = h2f(hw0 & 0xFFFFu), dmin = h2f(hw0 >> 16);
        const uint8_t bq = (l < 16 ? m.q + ui * 16 : m.q + m.plane + ui * 16)[l & 15];
        const bool hi = g & 1;
        const float d1 = d * (float)(hi ? sc1 : sc0), mm = dmin * (float)(hi ? m1 : m0);
        return d1 * (float)(hi ? (bq >> 4) : (bq & 15)) - mm;
    }
    case T_Q6_K: {
        const int sb = col >> 8, w = col & 255, h = w >> 7, rr = w & 127, k = rr >> 5, l = rr & 31;
        const int l0 = l & 16, bi = l & 15;
        const size_t ui = (size_t)row * (m.cols >> 6) + 4 * sb + 2 * h + (l0 >> 4);
        const size_t sbi = (size_t)row * (m.cols >> 8) + sb;
        const uint8_t qlb = (k & 1 ? m.q + m.plane : m.q)[ui * 16 + bi];
        const uint8_t qhb = m.q[2 * m.plane + ui * 16 + bi];
        const int q = (int)(((k < 2 ? qlb & 15 : qlb >> 4)) | (((qhb >> (2 * k)) & 3) << 4)) - 32;
        const int8_t sc = ((const int8_t *)(m.s + sbi * 16))[8 * h + (l >> 4) + 2 * k];
        return h2f(m.d[sbi]) * (float)sc * (float)q;
    }
    case T_Q8_0: {
        const size_t ui = (size_t)row * (m.cols >> 6) + (col >> 6);
        const int c = (col >> 4) & 3;
        const float d = h2f(m.d[(size_t)row * (m.cols >> 5) + (col >> 5)]);
        return d * (float)((const int8_t *)(m.q + c * m.plane + ui * 16))[col & 15];
    }
    case T_F16: return h2f(((const uint16_t *)m.q)[(size_t)row * m.cols + col]);
    default: return ((const float *)m.q)[(size_t)row * m.cols + col];
    }
}

// ------------------------------------------------------------- attention --
// Per half workgroup (4 compute waves), LDS scratch for head_dim 128, G <= 4.
constexpr int AHD = 128;
constexpr int AG = 4;
constexpr int PST = AHD + 4;  // floats per attention partial: o[AHD], m, l, 2 pad (16-byte rows)
struct __attribute__((aligned(16))) AttnLds {
    float qr[AG][AHD];      // raw q heads (I/O wave)
    float qT[AHD][AG];      // normalized + rotated q, [dim][head]
    float kp[AHD], vp[AHD], qn[AHD], kn[AHD];
    float2 cs[AHD / 2];
    uint16_t kpos[AHD], vpos[AHD];
    float sp[4][AG][64];    // per-wave partial scores
    float pT[64][AG];       // softmax numerators, [position][head]
    float ob[4][AG][AHD];
    float mx[AG], sm[AG], nrm[AG + 1];
};

struct KVReg {
    u32x4 k[4];
    uint32_t v[16];
};

// chunk index of round `rd` for half `h` of this workgroup; -1 if none
static __device__ __forceinline__ int attn_chunk_of(const StreamArgs &a, int h, int rd, int nchunk, int &kvh) {
    const int slot = 2 * blockIdx.x + h, spk = 2 * a.G / a.n_kv;
    kvh = slot % a.n_kv;
    const int c = slot / a.n_kv + rd * spk;
    return c < nchunk ? c : -1;
}

// K/V tile loads of chunk c for thread (wave w of the half, lane l):
// K row t0 + l, dims [32w, 32w+32); V rows t0 + 16w + i, dims 2l, 2l+1
#if defined(__HIP_DEVICE_COMPILE__)
#define GLB(T, p) ((const __attribute__((address_space(1))) T *)(p))
#else
#define GLB(T, p) ((const T *)(p))
#endif
static __device__ __forceinline__ void attn_issue(const StreamArgs &a, const SLayer &L, int kvh, int c, int pos,
                                                  KVReg &kv) {
    const int w = (threadIdx.x >> 6) & 3, lane = threadIdx.x & 63;
    const int t0 = 64 * c, n = min(64, pos + 1 - t0);
    const uint16_t *kc = L.kc + (size_t)kvh * a.seq_len * AHD, *vc = L.vc + (size_t)kvh * a.seq_len * AHD;
    const auto kr = GLB(u32x4, kc + (size_t)(t0 + min(lane, n - 1)) * AHD + 32 * w);
#pragma unroll
    for (int i = 0; i < 4; i++) kv.k[i] = __builtin_nontemporal_load(kr + i);
#pragma unroll
    for (int i = 0; i < 16; i++)
        kv.v[i] = __builtin_nontemporal_load(GLB(uint32_t, vc + (size_t)(t0 + min(16 * w + i, n - 1)) * AHD) + lane);
}

// ------------------------------------------------------------------ kernel --
// The two roles run the same sequence of workgroup barriers (__syncthreads):
// per stage, A (inputs in LDS) and B (outputs in LDS); ATTN adds 3 for the
// head norm / RoPE and 4 per round.  The I/O wave waits for the grid barrier
// only before A; on a timeout it sets `abort`, which every wave checks after A.

struct Ctx {
    Lds s;
    uint64_t seq;
    int nb_total;
};

static __device__ __forceinline__ Ctx make_ctx(const StreamArgs &a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    Ctx c;
    c.s.ring = smem;
    c.s.xr = smem + S_NCW * S_RING_BYTES;
    const int kmax = max(a.D, max(a.H, a.QD));
    const int xbytes = max((int)((qvec_bytes(kmax) + 1023) & ~1023), (int)(2 * sizeof(AttnLds)));
    c.s.misc = (Misc *)(c.s.xr + ((xbytes + 15) & ~15));
    c.s.yo = (float *)(c.s.misc + 1);
    c.nb_total = 1 + 6 * a.n_layers;
    c.seq = *(const uint64_t *)(a.state + ST_SEQ);
    return c;
}

static __device__ __forceinline__ int attn_rounds(const StreamArgs &a, int nchunk) {
    const int spk = 2 * a.G / a.n_kv;
    return (nchunk + spk - 1) / spk;
}

// ------------------------------------------------------------- I/O wave --
static __device__ void io_main(const StreamArgs &a, const Ctx &cx) {
    const int lane = threadIdx.x & 63, wg = blockIdx.x, G = a.G;
    const Lds &s = cx.s;
    Misc &ms = *s.misc;
    const uint64_t seq = cx.seq;
    const int nbt = cx.nb_total;
    int stage = 0;
    uint32_t bt = 0;  // barrier target
    // wait for the barrier of the previous stage; false: abort the launch
    auto wait_prev = [&]() -> bool {
        if (grid_wait(a, seq, nbt, stage - 1)) {
            TRACE(a, stage, 0);
            return true;
        }
        if (lane == 0) {
            ms.abort = 1;
            st_i(a.state + ST_ERR, S_ERR_TIMEOUT);
        }
        return false;
    };
    auto arrive = [&]() {
        vm_wait_all();  // this workgroup's stores are complete
        TRACE(a, stage, 6);
        grid_arrive(a);
    };

    // EMBED: token (argmax of the previous launch if pending), this
    // workgroup's rows of x = token_embd[token] (forward.odin:72-75)
    int token = a.state[ST_TOKEN], pos = a.state[ST_POS];
    const bool pending = a.state[ST_PENDING] != 0;
    if (pending) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
        for (int i = lane; i < G; i += 64)
            if (better(a.am_val[i], a.am_idx[i], bv, bi)) {
                bv = a.am_val[i];
                bi = a.am_idx[i];
            }
        wave_best(bv, bi);
        token = bi == 0x7FFFFFFF ? 0 : bi;
        pos += 1;
    }
    if (token < 0 || token >= a.vocab) token = 0;
    if (lane == 0) {
        ms.token = token;
        ms.pos = pos;
        ms.abort = 0;
        ms.kv_store[0] = ms.kv_store[1] = 0;
    }
    {
        const int r0 = wg * a.rD, n = max(0, min(a.rD, a.D - r0));
        for (int i = lane; i < n; i += 64) ms.xres[i] = emb_elem(a.emb, token, r0 + i);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (n > 0) {
            const float ss = io_quantize(ms.xres, a.layers[0].attn_norm + r0, n, r0, a.D, a.xq, ms.qstage);
            if (lane == 0) st_f(a.ssq + wg, ss);
        }
    }
    arrive();
    stage++;
    const int nchunk = pos / 64 + 1;
    const int Gq = a.n_heads / a.n_kv;

    for (int l = 0; l < a.n_layers; l++) {
        const SLayer &L = a.layers[l];
        // ------------------------------------------------------- QKV --
        if (wait_prev()) {
            io_dma(a.xq, s.xr, (int)qvec_bytes(a.D));
            const float sc = io_norm_scale(a);
            vm_wait_all();
            if (lane == 0) ms.s_norm = sc;
            if (wg == 0 && l == 0 && lane == 0) {  // every workgroup has read the state: publish this step
                int32_t *st = a.state;
                if (pending) {
                    const int step = st[ST_STEP];
                    if (a.tokens && step >= 0 && step < st[ST_CAP]) st_i(a.tokens + step, token);
                    st_i(st + ST_STEP, step + 1);
                    st_i(st + ST_PENDING, 0);
                }
                st_i(st + ST_TOKEN, token);
                st_i(st + ST_POS, pos);
            }
        }
        TRACE(a, stage, 1);
        lds_bar(&ms.bar, bt);  // A
        if (ms.abort) return;
        lds_bar(&ms.bar, bt);  // B
        TRACE(a, stage, 5);
        {
            const SWgRows wr = a.wgrows[(size_t)L.plan[SK_QKV] * G + wg];
            for (int v = wr.v0 + lane; v < wr.v1; v += 64) {
                const float y = s.yo[v - wr.v0];
                if (v < a.QD) st_f(a.q + v, y);
                else if (v < a.QD + a.KVD) st_f(a.k + (v - a.QD), y);
                else st_f(a.v + (v - a.QD - a.KVD), y);
            }
        }
        lds_bar(&ms.bar, bt);  // C: the stores are issued ahead of the compute waves' K/V tile loads
        arrive();
        stage++;

        // ------------------------------------------------------ ATTN --
        AttnLds *al = (AttnLds *)s.xr;
        // the head norms and the RoPE row of pos (read-only: requested before
        // the barrier; the QKV input in this LDS area is no longer read)
        for (int h = 0; h < 2; h++) {
            AttnLds &A = al[h];
            io_dma_half((const uint8_t *)L.q_norm, (uint8_t *)A.qn, 0);
            io_dma_half((const uint8_t *)L.k_norm, (uint8_t *)A.kn, 0);
            io_dma_half((const uint8_t *)(a.rope_cs + (size_t)pos * (AHD / 2)), (uint8_t *)A.cs, 0);
        }
        if (wait_prev()) {
            // this token's q heads, k and v of each half's KV head (device-scope
            // direct-to-LDS loads)
            for (int h = 0; h < 2; h++) {
                int kvh;
                attn_chunk_of(a, h, 0, 1 << 30, kvh);
                AttnLds &A = al[h];
                io_dma((const uint8_t *)(a.q + (size_t)kvh * Gq * AHD), (uint8_t *)A.qr, Gq * AHD * 4);
                io_dma_half((const uint8_t *)(a.k + (size_t)kvh * AHD), (uint8_t *)A.kp, 16);
                io_dma_half((const uint8_t *)(a.v + (size_t)kvh * AHD), (uint8_t *)A.vp, 16);
            }
            vm_wait_all();
        }
        TRACE(a, stage, 1);
        lds_bar(&ms.bar, bt);  // A
        if (ms.abort) return;
        lds_bar(&ms.bar, bt);  // head norms
        lds_bar(&ms.bar, bt);  // RoPE
        lds_bar(&ms.bar, bt);  // f16 k/v of pos
        const int rounds = attn_rounds(a, nchunk);
        for (int rd = 0; rd < rounds; rd++) {
            lds_bar(&ms.bar, bt);  // scores
            lds_bar(&ms.bar, bt);  // softmax
            lds_bar(&ms.bar, bt);  // o partials
            lds_bar(&ms.bar, bt);  // o reduced
            for (int h = 0; h < 2; h++) {  // partials of both halves, and K/V[pos]
                int kvh;
                const int ch = attn_chunk_of(a, h, rd, nchunk, kvh);
                if (ch < 0) continue;
                const AttnLds &B = al[h];
                for (int g = 0; g < Gq; g++) {
                    float *pp = a.part + ((size_t)(kvh * Gq + g) * a.max_chunks + ch) * PST;
                    for (int i = lane; i < AHD; i += 64) st_f(pp + i, B.ob[0][g][i]);
                    if (lane == 0) {
                        st_f(pp + AHD, B.mx[g]);
                        st_f(pp + AHD + 1, B.sm[g]);
                    }
                }
                if (pos >= 64 * ch && pos < 64 * ch + 64) {  // this chunk holds pos: store K/V[pos] (f16)
                    uint32_t *kd = (uint32_t *)(L.kc + ((size_t)kvh * a.seq_len + pos) * AHD);
                    uint32_t *vd = (uint32_t *)(L.vc + ((size_t)kvh * a.seq_len + pos) * AHD);
                    for (int i = lane; i < AHD / 2; i += 64) {
                        kd[i] = *(const uint32_t *)&B.kpos[2 * i];
                        vd[i] = *(const uint32_t *)&B.vpos[2 * i];
                    }
                }
            }
        }
        arrive();
        stage++;

        // ------------------------------------------------------ COMB --
        if (wait_prev()) {
            // this workgroup's rQ dims of att, 16 at a time (one head each):
            // O = sum_c exp(m_c - M) o_c / sum_c exp(m_c - M) l_c over the chunks
            const int e0 = wg * a.rQ, n = max(0, min(a.rQ, a.QD - e0));
            float *cb = (float *)s.xr;  // [pass of 64 chunks][5][64 lanes][4]: o[d0..d0+16), (m, l, -, -)
            for (int b0 = 0; b0 < n; b0 += 16) {
                const int e = e0 + b0, hh = e / AHD, d0 = e % AHD;
                const float *pb = a.part + (size_t)hh * a.max_chunks * PST;
                const int npass = (nchunk + 63) / 64;
                for (int ps = 0; ps < npass; ps++) {
                    const int cc = min(ps * 64 + lane, nchunk - 1);
                    const float *pc = pb + (size_t)cc * PST;
                    for (int q = 0; q < 4; q++)
                        __builtin_amdgcn_global_load_lds((const void *)(pc + d0 + 4 * q), LDS_PTR(cb + (ps * 5 + q) * 256),
                                                         16, 0, 16);
                    __builtin_amdgcn_global_load_lds((const void *)(pc + AHD), LDS_PTR(cb + (ps * 5 + 4) * 256), 16, 0,
                                                     16);
                }
                vm_wait_all();
                float M = -INFINITY;
                for (int ps = 0; ps < npass; ps++)
                    if (ps * 64 + lane < nchunk) M = fmaxf(M, cb[(ps * 5 + 4) * 256 + 4 * lane]);
                M = wave_max(M);
                float Ls = 0.f, O[16];
#pragma unroll
                for (int i = 0; i < 16; i++) O[i] = 0.f;
                for (int ps = 0; ps < npass; ps++) {
                    if (ps * 64 + lane >= nchunk) continue;
                    const float f = expf(cb[(ps * 5 + 4) * 256 + 4 * lane] - M);
                    Ls += f * cb[(ps * 5 + 4) * 256 + 4 * lane + 1];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 o4 = *(const float4 *)(cb + (ps * 5 + q) * 256 + 4 * lane);
                        O[4 * q] += f * o4.x;
                        O[4 * q + 1] += f * o4.y;
                        O[4 * q + 2] += f * o4.z;
                        O[4 * q + 3] += f * o4.w;
                    }
                }
                Ls = wave_sum(Ls);
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float oi = wave_sum(O[i]);
                    if (lane == i) s.yo[b0 + i] = oi / Ls;
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (n > 0) io_quantize(s.yo, nullptr, n, e0, a.QD, a.attq, ms.qstage);
            arrive();
        }
        TRACE(a, stage, 1);
        lds_bar(&ms.bar, bt);  // A
        if (ms.abort) return;
        stage++;

        // -------------------------------------------------------- WO --
        {  // ffn_norm rows for this stage's epilogue: requested now, complete with the gather
            const int r0 = wg * a.rD, n = max(0, min(a.rD, a.D - r0));
            io_dma((const uint8_t *)(L.ffn_norm + r0), (uint8_t *)ms.nrm, 4 * n);
        }
        if (wait_prev()) {
            io_dma(a.attq, s.xr, (int)qvec_bytes(a.QD));
            vm_wait_all();
        }
        TRACE(a, stage, 1);
        lds_bar(&ms.bar, bt);  // A
        if (ms.abort) return;
        lds_bar(&ms.bar, bt);  // B
        TRACE(a, stage, 5);
        {
            const int r0 = wg * a.rD, n = max(0, min(a.rD, a.D - r0));
            for (int i = lane; i < n; i += 64) ms.xres[i] = ms.xres[i] + s.yo[i];  // forward.odin:117-121
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (n > 0) {
                const float ss = io_quantize(ms.xres, ms.nrm, n, r0, a.D, a.xq, ms.qstage);
                if (lane == 0) st_f(a.ssq + wg, ss);
            }
        }
        arrive();
        stage++;

        // -------------------------------------------------------- GU --
        if (wait_prev()) {
            io_dma(a.xq, s.xr, (int)qvec_bytes(a.D));
            const float sc = io_norm_scale(a);
            vm_wait_all();
            if (lane == 0) ms.s_norm = sc;
        }
        TRACE(a, stage, 1);
        lds_bar(&ms.bar, bt);  // A
        if (ms.abort) return;
        lds_bar(&ms.bar, bt);  // B
        TRACE(a, stage, 5);
        {
            const int r0 = wg * a.rH, n = max(0, min(a.rH, a.H - r0));
            if (n > 0) io_quantize(s.yo, nullptr, n, r0, a.H, a.hbq, ms.qstage);
        }
        arrive();
        stage++;

        // ------------------------------------------------------ DOWN --
        {  // the next norm's rows (next layer's attn_norm, or output_norm)
            const int r0 = wg * a.rD, n = max(0, min(a.rD, a.D - r0));
            const float *nw = l + 1 < a.n_layers ? a.layers[l + 1].attn_norm : a.output_norm;
            io_dma((const uint8_t *)(nw + r0), (uint8_t *)ms.nrm, 4 * n);
        }
        if (wait_prev()) {
            io_dma(a.hbq, s.xr, (int)qvec_bytes(a.H));
            vm_wait_all();
        }
        TRACE(a, stage, 1);
        lds_bar(&ms.bar, bt);  // A
        if (ms.abort) return;
        lds_bar(&ms.bar, bt);  // B
        TRACE(a, stage, 5);
        {
            const int r0 = wg * a.rD, n = max(0, min(a.rD, a.D - r0));
            for (int i = lane; i < n; i += 64) ms.xres[i] = ms.xres[i] + s.yo[i];  // forward.odin:134-139
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (n > 0) {
                const float ss = io_quantize(ms.xres, ms.nrm, n, r0, a.D, a.xq, ms.qstage);
                if (lane == 0) st_f(a.ssq + wg, ss);
            }
        }
        arrive();
        stage++;
    }

    // ------------------------------------------------------------ VOCAB --
    if (wait_prev()) {
        io_dma(a.xq, s.xr, (int)qvec_bytes(a.D));
        const float sc = io_norm_scale(a);
        vm_wait_all();
        if (lane == 0) ms.s_norm = sc;
    }
    TRACE(a, stage, 1);
    lds_bar(&ms.bar, bt);  // A
    if (ms.abort) return;
    lds_bar(&ms.bar, bt);  // B
    TRACE(a, stage, 5);
    const SWgRows wr = a.wgrows[(size_t)a.vocab_plan * G + wg];
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int v = wr.v0 + lane; v < wr.v1; v += 64) {
        const float y = s.yo[v - wr.v0];
        a.logits[v] = y;
        if (better(y, v, bv, bi)) {
            bv = y;
            bi = v;
        }
    }
    wave_best(bv, bi);
    if (lane == 0) {
        a.am_val[wg] = bv;
        a.am_idx[wg] = bi;
        if (wg == 0) {
            a.state[ST_PENDING] = 1;
            *(uint64_t *)(a.state + ST_SEQ) = seq + 1;
        }
    }
}

// --------------------------------------------------------- compute waves --
static __device__ void attn_compute(const StreamArgs &a, const SLayer &L, const Ctx &cx, int wave, int pos,
                                    int nchunk, KVReg (&kvr)[2], uint32_t &bt) {
    const int tid = threadIdx.x, lane = tid & 63, half = wave >> 2, tw = wave & 3, th = tid & 255;
    Misc &ms = *cx.s.misc;
    AttnLds &A = ((AttnLds *)cx.s.xr)[half];
    const int Gq = a.n_heads / a.n_kv;
    // q heads and k: RMSNorm (ops.odin:7-19), then RoPE (forward.odin:117-145)
    for (int g = tw; g < Gq + 1; g += 4) {
        const float *src = g < Gq ? A.qr[g] : A.kp;
        float ss = 0.f;
        for (int i = lane; i < AHD; i += 64) ss += src[i] * src[i];
        ss = wave_sum(ss);
        if (lane == 0) A.nrm[g] = 1.0f / sqrtf(ss / (float)AHD + a.eps);
    }
    lds_bar(&ms.bar, bt);  // head norms
    for (int idx = th; idx < AG * (AHD / 2); idx += 256) {
#pragma clang fp contract(off)
        const int g = idx / (AHD / 2), i = idx % (AHD / 2);
        if (g < Gq) {
            const float sn = A.nrm[g];
            const float x = A.qn[i] * (sn * A.qr[g][i]);
            const float y = A.qn[i + AHD / 2] * (sn * A.qr[g][i + AHD / 2]);
            const float c = A.cs[i].x, sg = A.cs[i].y;
            A.qT[i][g] = x * c - y * sg;
            A.qT[i + AHD / 2][g] = x * sg + y * c;
        } else {  // unused head slots stay zero
            A.qT[i][g] = 0.f;
            A.qT[i + AHD / 2][g] = 0.f;
        }
    }
    if (th < AHD / 2) {
#pragma clang fp contract(off)
        const int i = th;
        const float sn = A.nrm[Gq];
        const float x = A.kn[i] * (sn * A.kp[i]);
        const float y = A.kn[i + AHD / 2] * (sn * A.kp[i + AHD / 2]);
        const float c = A.cs[i].x, sg = A.cs[i].y;
        // K/V[pos] as stored in the f16 cache (infer/metal.odin:443-454)
        A.kpos[i] = f2h(x * c - y * sg);
        A.kpos[i + AHD / 2] = f2h(x * sg + y * c);
        A.vpos[i] = f2h(A.vp[i]);
        A.vpos[i + AHD / 2] = f2h(A.vp[i + AHD / 2]);
    }
    lds_bar(&ms.bar, bt);  // RoPE
    lds_bar(&ms.bar, bt);  // (kept: the I/O wave mirrors three barriers here)
    const int rounds = attn_rounds(a, nchunk);
    for (int rd = 0; rd < rounds; rd++) {
        int kvh;
        const int c = attn_chunk_of(a, half, rd, nchunk, kvh);
        KVReg &kv = kvr[rd & 1];  // rounds rd and rd+1 were requested before this one
        const int t0 = 64 * max(c, 0), n = c >= 0 ? min(64, pos + 1 - t0) : 0;
        // scores: thread (tw, lane) = position t0 + lane, dims [32 tw, 32 tw + 32)
        if (c >= 0) {
            float acc[AG] = {0.f, 0.f, 0.f, 0.f};
            const bool at_pos = t0 + lane == pos;
#pragma unroll 1
            for (int i = 0; i < 4; i++) {
                const u32x4 kw = at_pos ? *(const u32x4 *)&A.kpos[32 * tw + 8 * i] : kv.k[i];
                const uint32_t ws[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float kk = h2f((ws[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
                    const float4 q4 = *(const float4 *)A.qT[32 * tw + 8 * i + e];
                    acc[0] += q4.x * kk;
                    acc[1] += q4.y * kk;
                    acc[2] += q4.z * kk;
                    acc[3] += q4.w * kk;
                }
            }
#pragma unroll
            for (int g = 0; g < AG; g++)
                if (g < Gq) A.sp[tw][g][lane] = acc[g];
        }
        lds_bar(&ms.bar, bt);  // scores
        if (c >= 0) {     // split-local softmax (ops.odin:21-37), one wave per head
            const float div = sqrtf((float)AHD);
            for (int g = tw; g < AG; g += 4) {
                const int t = lane;
                float e = 0.f;
                if (g < Gq) {
                    const float sc = t < n ? ((A.sp[0][g][t] + A.sp[1][g][t]) + (A.sp[2][g][t] + A.sp[3][g][t])) / div
                                           : -INFINITY;
                    const float m = wave_max(sc);
                    e = t < n ? expf(sc - m) : 0.f;
                    const float lsum = wave_sum(e);
                    if (lane == 0) {
                        A.mx[g] = m;
                        A.sm[g] = lsum;
                    }
                }
                A.pT[t][g] = e;
            }
        }
        lds_bar(&ms.bar, bt);  // softmax
        // o = sum_t p(t) v(t): thread (tw, lane) = positions 16 tw .. +15, dims 2 lane, 2 lane + 1
        if (c >= 0) {
            float o0[AG] = {0.f, 0.f, 0.f, 0.f}, o1[AG] = {0.f, 0.f, 0.f, 0.f};
            const uint32_t vpw = *(const uint32_t *)&A.vpos[2 * lane];
#pragma unroll 4
            for (int i = 0; i < 16; i++) {
                const int t = 16 * tw + i;
                const uint32_t vw = t0 + t == pos ? vpw : kv.v[i];
                const float v0 = h2f(vw & 0xFFFFu), v1 = h2f(vw >> 16);
                const float4 p4 = *(const float4 *)A.pT[t];
                o0[0] += p4.x * v0;
                o1[0] += p4.x * v1;
                o0[1] += p4.y * v0;
                o1[1] += p4.y * v1;
                o0[2] += p4.z * v0;
                o1[2] += p4.z * v1;
                o0[3] += p4.w * v0;
                o1[3] += p4.w * v1;
            }
#pragma unroll
            for (int g = 0; g < AG; g++)
                if (g < Gq) {
                    A.ob[tw][g][2 * lane] = o0[g];
                    A.ob[tw][g][2 * lane + 1] = o1[g];
                }
        }
        {  // round rd + 2 reuses this round's registers
            int kvh2;
            const int c2 = attn_chunk_of(a, half, rd + 2, nchunk, kvh2);
            if (c2 >= 0) attn_issue(a, L, kvh2, c2, pos, kv);
        }
        lds_bar(&ms.bar, bt);  // o partials
        if (c >= 0)
            for (int idx = th; idx < Gq * AHD; idx += 256) {
                const int g = idx / AHD, i = idx % AHD;
                A.ob[0][g][i] = (A.ob[0][g][i] + A.ob[1][g][i]) + (A.ob[2][g][i] + A.ob[3][g][i]);
            }
        lds_bar(&ms.bar, bt);  // o reduced
    }
}

// Stage program of the compute waves: per layer QKV, ATTN, COMB, WO, GU,
// DOWN, then VOCAB; one GEMV call site for all weight stages.
static __device__ void compute_main(const StreamArgs &a, const Ctx &cx, int wave) {
    const int cw = blockIdx.x * S_NCW + wave;
    const Lds &s = cx.s;
    Misc &ms = *s.misc;
    uint32_t bt = 0;  // barrier target
    Ring r;
    r.consumed = 0;
    r.lds = s.ring + wave * S_RING_BYTES;
    r.filled = &ms.filled[wave];
    r.consumed_p = &ms.consumed[wave];
    r.allow_p = &ms.allow[wave];
    r.abort_p = (uint32_t *)&ms.abort;
    r.err_p = a.state + ST_ERR;
    r.trace = a.trace != nullptr;
    r.wait_ticks = 0;
    uint32_t soff = 0;
    const int nst = 6 * a.n_layers + 1;
    for (int st = 0; st < nst; st++) {
        const int l = st / 6, k = st % 6;  // k: 0 QKV, 1 ATTN, 2 COMB, 3 WO, 4 GU, 5 DOWN; l == n_layers: VOCAB
        const bool voc = l == a.n_layers;
        const int pos = ms.pos, nchunk = pos / 64 + 1;
        if (k == 1 && !voc) {
            // the K/V tiles of the first round do not depend on this token:
            // requested while the I/O wave waits for the QKV results
            KVReg kv[2];
            for (int rd = 0; rd < 2; rd++) {
                int kvh;
                const int c0 = attn_chunk_of(a, wave >> 2, rd, nchunk, kvh);
                if (c0 >= 0) attn_issue(a, a.layers[l], kvh, c0, pos, kv[rd]);
            }
            lds_bar(&ms.bar, bt);  // A
            if (ms.abort) break;
            if (wave == 0) TRACE(a, st + 1, 2);
            attn_compute(a, a.layers[l], cx, wave, pos, nchunk, kv, bt);
            if (wave == 0) TRACE(a, st + 1, 4);
            continue;
        }
        // the stage's plan tables, requested before the barrier wait so the
        // loads after it hit the scalar cache
        const int pl = (k == 2 && !voc) ? -1 : voc ? a.vocab_plan : CST(a.layers)[l].plan[k == 0 ? SK_QKV : k - 2];
        int touch = 0;
        if (pl >= 0) {
            const auto *kp = CST(a.kinds) + pl;
            const auto *wp = CST(a.waves) + (size_t)pl * a.G * S_NCW + cw;
            touch = kp->nseg + kp->seg[2].rows + wp->nruns + wp->run[S_MAXRUN - 1].nrows +
                    CST(a.wgrows)[(size_t)pl * a.G + blockIdx.x].v0;
        }
        lds_bar(&ms.bar, bt);  // A
        if (ms.abort) break;
        if (wave == 0) TRACE(a, st + 1, 2);
        if (k == 2 && !voc) continue;
        if (touch == INT32_MIN) break;  // never: keeps the early loads
        const float scale = (voc || k == 0 || k == 4) ? ms.s_norm : 1.0f;
        gemv_stage(a, cw, r, soff, pl, s.xr, s.yo, scale, st + 1);
        if (wave == 0) TRACE(a, st + 1, 4);
        TRACE_SET(a, st + 1, 8 + wave, r.wait_ticks);
        r.wait_ticks = 0;
        lds_bar(&ms.bar, bt);  // B
        if (k == 0 && !voc) lds_bar(&ms.bar, bt);  // C (QKV): the I/O wave's stores go first
    }
}

// ---------------------------------------------------------- loader waves --
// Loader L fills the rings of compute waves LS*L .. LS*L + LS-1 (LS =
// LSTREAMS) with 16-byte nontemporal loads: one wave instruction moves a
// 1 KB piece.  Its registers hold NGRP groups of LS slots, slot j of a group
// being one chunk (CP pieces) of stream j.  The groups are handled in turn:
// a group's chunks are written to the rings (one LDS wait, then the fill
// counters), and each slot is refilled with the next chunk of its stream if
// the ring has room for it (piece p may be loaded once the compute wave has
// consumed piece p - S_RING).  The other groups' loads stay in flight
// meanwhile.  A slot with nothing to load re-reads a small resident buffer
// (the data is dropped), so the count of loads in flight stays exact.
// Streams are padded to whole chunks (wstride is a multiple of 4 KB); pieces
// past a stream's end land in ring slots its compute wave no longer reads.
constexpr int LSTREAMS = S_NCW / S_NLD;
constexpr int CP = S_CP;
constexpr int NGRP = 4;

static __device__ __forceinline__ void loader_main(const StreamArgs &a, const Ctx &cx, int L) {
    const int lane = threadIdx.x & 63;
    Misc &ms = *cx.s.misc;
    const int w0 = L * LSTREAMS;
    const u32x4 *base[LSTREAMS];
    uint32_t n[LSTREAMS], issued[LSTREAMS];  // pieces of the stream, chunks requested
#pragma unroll
    for (int j = 0; j < LSTREAMS; j++) {
        const int cw = blockIdx.x * S_NCW + w0 + j;
        base[j] = (const u32x4 *)(a.wstream + (size_t)cw * a.wstride) + lane;
        n[j] = uni((uint32_t)CST(a.wpieces)[cw]);
        issued[j] = 0;
    }
    const u32x4 *dummy = (const u32x4 *)a.xq + lane;
    u32x4 data[NGRP][LSTREAMS][CP];
    uint32_t sc[NGRP][LSTREAMS];  // chunk + 1 held by the slot, 0: none
#pragma unroll
    for (int g = 0; g < NGRP; g++)
#pragma unroll
        for (int j = 0; j < LSTREAMS; j++) {
#pragma unroll
            for (int k = 0; k < CP; k++) data[g][j][k] = __builtin_nontemporal_load(dummy);
            sc[g][j] = 0;
        }
    const uint32_t *abort_p = (const uint32_t *)&ms.abort;
    uint32_t n_real = 0, n_idle = 0, n_sleep = 0;  // debugging counts
    while (true) {
        bool any = false;
#pragma unroll
        for (int g = 0; g < NGRP; g++) {
            bool ret = false;
#pragma unroll
            for (int j = 0; j < LSTREAMS; j++)
                if (sc[g][j]) {
                    uint8_t *ring = cx.s.ring + (w0 + j) * S_RING_BYTES + lane * 16;
                    const uint32_t p0 = (sc[g][j] - 1) * CP;
#pragma unroll
                    for (int k = 0; k < CP; k++) *(u32x4 *)(ring + ((p0 + k) % S_RING) * 1024) = data[g][j][k];
                    ret = true;
                }
            if (ret) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (lane == 0) {
#pragma unroll
                    for (int j = 0; j < LSTREAMS; j++)
                        if (sc[g][j]) lds_st(&ms.filled[w0 + j], sc[g][j] * CP);
                }
                any = true;
            }
            uint32_t cons[LSTREAMS];
#pragma unroll
            for (int j = 0; j < LSTREAMS; j++) cons[j] = lds_ld(&ms.consumed[w0 + j]);
            uint32_t allow[LSTREAMS];
#pragma unroll
            for (int j = 0; j < LSTREAMS; j++) allow[j] = lds_ld(&ms.allow[w0 + j]);
#pragma unroll
            for (int j = 0; j < LSTREAMS; j++) {
                const uint32_t c = issued[j];
                const bool ok =
                    uni(c * CP < n[j] && (c + 1) * CP <= min(cons[j] / 1024 + S_RING, allow[j] + CP - 1));
                const u32x4 *src = ok ? base[j] + (size_t)c * (CP * 64) : dummy;
#pragma unroll
                for (int k = 0; k < CP; k++) data[g][j][k] = __builtin_nontemporal_load(ok ? src + k * 64 : dummy);
                sc[g][j] = ok ? c + 1 : 0;
                issued[j] = c + (ok ? 1 : 0);
                any = any || ok;
                n_real += ok ? 1 : 0;
                n_idle += ok ? 0 : 1;
            }
        }
        if (!any) {
            bool done = true;
#pragma unroll
            for (int j = 0; j < LSTREAMS; j++) done = done && issued[j] * CP >= n[j];
            if (done || lds_ld(abort_p)) break;
            __builtin_amdgcn_s_sleep(2);  // all rings full: let the compute waves catch up
            n_sleep++;
        }
        if (lds_ld(abort_p)) break;
    }
    vm_wait_all();
    TRACE_SET(a, 6 * a.n_layers + 1, 16 + 4 * L, n_real);
    TRACE_SET(a, 6 * a.n_layers + 1, 17 + 4 * L, n_idle);
    TRACE_SET(a, 6 * a.n_layers + 1, 18 + 4 * L, n_sleep);
}

__global__ __launch_bounds__(S_THREADS) void stream_kernel(StreamArgs a) {
    const Ctx cx = make_ctx(a);
    const int wave = (int)uni(threadIdx.x >> 6);  // wave-uniform: the role branch is scalar
    if (threadIdx.x < S_NCW) {
        cx.s.misc->filled[threadIdx.x] = 0;
        cx.s.misc->consumed[threadIdx.x] = 0;
        cx.s.misc->allow[threadIdx.x] = S_LEAD;
    }
    if (threadIdx.x == 0) {
        cx.s.misc->bar = 0;
        cx.s.misc->abort = 0;
    }
    __syncthreads();  // the only barrier of all waves: the counters above are set
    if (wave == NTOT_IO) {
        io_main(a, cx);
        vm_wait_all();
    } else if (wave >= S_NCW) {
        loader_main(a, cx, wave - S_NCW);
    } else {
        compute_main(a, cx, wave);
    }
}

// reduce the pending argmax partials of the last launch into the state and
// the token list (the next launch would do it at its start)
__global__ __launch_bounds__(64) void stream_finalize_kernel(StreamArgs a) {
    const int lane = threadIdx.x;
    if (!a.state[ST_PENDING]) return;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = lane; i < a.G; i += 64)
        if (better(a.am_val[i], a.am_idx[i], bv, bi)) {
            bv = a.am_val[i];
            bi = a.am_idx[i];
        }
    wave_best(bv, bi);
    if (lane == 0) {
        if (bi == 0x7FFFFFFF) bi = 0;
        const int step = a.state[ST_STEP];
        if (a.tokens && step >= 0 && step < a.state[ST_CAP]) a.tokens[step] = bi;
        a.state[ST_STEP] = step + 1;
        a.state[ST_TOKEN] = bi;
        a.state[ST_POS] = a.state[ST_POS] + 1;
        a.state[ST_PENDING] = 0;
    }
}

size_t stream_lds_bytes(int kmax, int yo_floats) {
    const size_t x = std::max((size_t)((qvec_bytes(kmax) + 1023) & ~1023), 2 * sizeof(AttnLds));
    return (size_t)S_NCW * S_RING_BYTES + ((x + 15) & ~(size_t)15) + sizeof(Misc) + (size_t)yo_floats * 4;
}

hipError_t launch_stream(const StreamArgs &a, hipStream_t st) {
    if (a.finalize_only) {
        hipLaunchKernelGGL(stream_finalize_kernel, dim3(1), dim3(64), 0, st, a);
        return hipGetLastError();
    }
    const size_t lds = stream_lds_bytes(std::max(a.D, std::max(a.H, a.QD)), a.yo_floats);
    static size_t set_for = 0;
    if (set_for < lds) {
        hipError_t e = hipFuncSetAttribute((const void *)stream_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) return e;
        set_for = lds;
    }
    StreamArgs b = a;
    void *args[] = {(void *)&b};
    return hipLaunchCooperativeKernel((const void *)stream_kernel, dim3(a.G), dim3(S_THREADS), args, (unsigned)lds, st);
}

}  // namespace oi
