// gemv.hip -- quantized GEMV for Q4_K, Q6_K and Q8_0 weights on gfx950
// (reference: infer/matmul.odin:77-109 over ggml/quant.odin:76-282), with the
// token loop's fusions: RMSNorm prologue (infer/ops.odin:7-19), residual add,
// SwiGLU (infer/forward.odin:128-132) and greedy-argmax partials
// (sampler/sampler.odin:79-89).
//
// Layout of the work:
//   * a row is cut into units of 64 weights; a lane owns units j, j+lpr, ...
//     of its row (lpr lanes per row, a power of two <= 64);
//   * a tile is R rows per lane group x (64/lpr) groups: one wave's rows;
//   * one workgroup of 16 waves per CU takes a contiguous range of tiles of
//     ONE segment (so one weight type per workgroup); its waves take the
//     tiles from a counter in LDS, request the weights of their first tile
//     before the x prologue, and double-buffer the rest in registers.
// Activations: x (after RMSNorm if asked) is quantized per 32 elements to a
// 22-bit integer q = 2^14*hi + 2^7*mid + lo (hi int8, mid and lo 0..127) with
// a float scale, so the products run on v_dot4_i32_i8 (three chains, one per
// byte plane); the result is scaled back in float.  The per-group x sums
// (exact float) serve the Q4_K min term and the Q6_K -32 offset.  The x
// rounding error is <= 2^-22 of the group maximum, below f32 accumulation
// noise, so greedy picks agree with an f32 reference down to ~1e-6 margins.

#include <algorithm>
#include <climits>

#include "device_common.h"

namespace oi {

constexpr float XQ_MAX = 2097151.0f;  // 2^21 - 1

static __device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// x in LDS: bytes of hi and lo in 16-byte chunks (16 elements); chunk C is
// stored at a slot that spreads the chunks read together over the banks.
static __device__ __forceinline__ int cslot(int C) { return (C & ~3) | ((C & 3) ^ ((C >> 4) & 3)); }

struct XQ {
    const u32x4 *hi, *mid, *lo;  // [K/16] chunks each
    const float *xs;       // [K/32] scale of the 15-bit integers
    const float *s32;      // [K/32] sums of x
    const float *s16;      // [K/16] sums of x
};

// ------------------------------------------------------------------ Q4_K --
struct WQ4K {
    u32x4 h, q0, q1;
};
static __device__ __forceinline__ void wload(const DMat &m, int row, int u, WQ4K &w) {
    const size_t ui = (size_t)row * (m.cols >> 6) + u;
    w.h = ldg_nt((const u32x4 *)(m.s + ((size_t)row * (m.cols >> 8) + (u >> 2)) * 16));
    w.q0 = ldg_nt((const u32x4 *)(m.q + ui * 16));
    w.q1 = ldg_nt((const u32x4 *)(m.q + m.plane + ui * 16));
}
struct XU4K {
    u32x4 h[4], m[4], l[4];
    float xs0, xs1, s0, s1;
};
static __device__ __forceinline__ void xload(const XQ &x, int u, XU4K &r) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        r.h[c] = x.hi[cslot(4 * u + c)];
        r.m[c] = x.mid[cslot(4 * u + c)];
        r.l[c] = x.lo[cslot(4 * u + c)];
    }
    r.xs0 = x.xs[2 * u];
    r.xs1 = x.xs[2 * u + 1];
    r.s0 = x.s32[2 * u];
    r.s1 = x.s32[2 * u + 1];
}
// the three byte-plane dot products of one 32-element group, combined
static __device__ __forceinline__ float plane_sum(int h, int m, int l) {
    return (float)h * 16384.f + ((float)m * 128.f + (float)l);
}

static __device__ __forceinline__ float wdot(const WQ4K &w, int u, const XU4K &x) {
    const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    int ah0 = 0, am0 = 0, al0 = 0, ah1 = 0, am1 = 0, al1 = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t lo = qw[k] & 0x0F0F0F0Fu, hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
        const int c0 = k >> 2, c1 = 2 + (k >> 2), e = k & 3;
        ah0 = sdot4(lo, x.h[c0][e], ah0);
        am0 = sdot4(lo, x.m[c0][e], am0);
        al0 = sdot4(lo, x.l[c0][e], al0);
        ah1 = sdot4(hi, x.h[c1][e], ah1);
        am1 = sdot4(hi, x.m[c1][e], am1);
        al1 = sdot4(hi, x.l[c1][e], al1);
    }
    const int p = u & 3;
    const float d = h2f(w.h.x & 0xFFFFu), dmin = h2f(w.h.x >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(p, w.h.y, w.h.z, w.h.w, sc0, m0, sc1, m1);
    // |ah| <= 32*15*128, so the 22-bit combination fits in int32
    const float q0 = (float)((ah0 << 14) + (am0 << 7) + al0) * x.xs0;
    const float q1 = (float)((ah1 << 14) + (am1 << 7) + al1) * x.xs1;
    return d * ((float)sc0 * q0 + (float)sc1 * q1) - dmin * ((float)m0 * x.s0 + (float)m1 * x.s1);
}

// ------------------------------------------------------------------ Q6_K --
struct WQ6K {
    u32x4 l0, l1, qh;
    u32x2 sc;
    uint32_t d;
};
static __device__ __forceinline__ void wload(const DMat &m, int row, int u, WQ6K &w) {
    const size_t sbi = (size_t)row * (m.cols >> 8) + (u >> 2);
    const size_t ui = (size_t)row * (m.cols >> 6) + u;
    const int h = (u >> 1) & 1;
    w.l0 = ldg_nt((const u32x4 *)(m.q + ui * 16));
    w.l1 = ldg_nt((const u32x4 *)(m.q + m.plane + ui * 16));
    w.qh = ldg_nt((const u32x4 *)(m.q + 2 * m.plane + ui * 16));
    w.sc = ldg_nt((const u32x2 *)(m.s + sbi * 16 + 8 * h));
    w.d = m.d[sbi];
}
// unit u covers elements e0 + 32k + [0,16), k = 0..3, e0 = 256 sb + 128 h + l0
struct XU6K {
    u32x4 h[4], m[4], l[4];
    float xs[4], s[4];
};
static __device__ __forceinline__ void xload(const XQ &x, int u, XU6K &r) {
    const int e0 = 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 16 * (u & 1);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int C = (e0 + 32 * k) >> 4;
        r.h[k] = x.hi[cslot(C)];
        r.m[k] = x.mid[cslot(C)];
        r.l[k] = x.lo[cslot(C)];
        r.xs[k] = x.xs[C >> 1];
        r.s[k] = x.s16[C];
    }
}
static __device__ __forceinline__ float wdot(const WQ6K &w, int u, const XU6K &x) {
    const uint32_t l0[4] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w};
    const uint32_t l1[4] = {w.l1.x, w.l1.y, w.l1.z, w.l1.w};
    const uint32_t qh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
    int ah[4] = {0, 0, 0, 0}, am[4] = {0, 0, 0, 0}, al[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // 6-bit values v = q + 32 (0..63) of the four sub-blocks, 4 per word
        const uint32_t v[4] = {(l0[i] & 0x0F0F0F0Fu) | ((qh[i] & 0x03030303u) << 4),
                               (l1[i] & 0x0F0F0F0Fu) | (((qh[i] >> 2) & 0x03030303u) << 4),
                               ((l0[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> 4) & 0x03030303u) << 4),
                               ((l1[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> 6) & 0x03030303u) << 4)};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            ah[k] = sdot4(v[k], x.h[k][i], ah[k]);
            am[k] = sdot4(v[k], x.m[k][i], am[k]);
            al[k] = sdot4(v[k], x.l[k][i], al[k]);
        }
    }
    const int bsh = (u & 1);  // scale byte (l0/16) + 2k of the 8 bytes of this half
    const uint32_t scw[2] = {w.sc.x, w.sc.y};
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int bi = bsh + 2 * k;
        const float s = (float)(int8_t)((scw[bi >> 2] >> ((bi & 3) * 8)) & 0xFFu);
        acc += s * (plane_sum(ah[k], am[k], al[k]) * x.xs[k] - 32.f * x.s[k]);
    }
    return h2f(w.d) * acc;
}

// ------------------------------------------------------------------ Q8_0 --
struct WQ80 {
    u32x4 q[4];
    uint32_t d;
};
static __device__ __forceinline__ void wload(const DMat &m, int row, int u, WQ80 &w) {
    const size_t ui = (size_t)row * (m.cols >> 6) + u;
#pragma unroll
    for (int c = 0; c < 4; c++) w.q[c] = ldg_nt((const u32x4 *)(m.q + c * m.plane + ui * 16));
    w.d = *(const uint32_t *)(m.d + 2 * ui);
}
static __device__ __forceinline__ float wdot(const WQ80 &w, int u, const XU4K &x) {
    int ah[2] = {0, 0}, am[2] = {0, 0}, al[2] = {0, 0};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int b = c >> 1;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            ah[b] = sdot4(w.q[c][e], x.h[c][e], ah[b]);
            am[b] = sdot4(w.q[c][e], x.m[c][e], am[b]);
            al[b] = sdot4(w.q[c][e], x.l[c][e], al[b]);
        }
    }
    return h2f(w.d & 0xFFFFu) * (plane_sum(ah[0], am[0], al[0]) * x.xs0) +
           h2f(w.d >> 16) * (plane_sum(ah[1], am[1], al[1]) * x.xs1);
}

template <int T> struct Types;
template <> struct Types<T_Q4_K> { using W = WQ4K; using X = XU4K; };
template <> struct Types<T_Q6_K> { using W = WQ6K; using X = XU6K; };
template <> struct Types<T_Q8_0> { using W = WQ80; using X = XU4K; };

// Quantize 4 consecutive values (one float4 per thread, 8 threads per group
// of 32) into the LDS layout.
static __device__ __forceinline__ void quant4(float4 v, int c, uint32_t *hw, uint32_t *mw, uint32_t *lw, float *xs,
                                              float *s32, float *s16) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    const float sum = (v.x + v.y) + (v.z + v.w);
    const float sum16 = dpp_sum4(sum);             // 4 lanes = 16 elements
    const float sum32 = sum16 + dpp_mirror8(sum16);  // 8 lanes = 32 elements
    amax = dpp_max8(amax);
    const float inv = amax > 0.f ? XQ_MAX / amax : 0.f;
    const int q0 = (int)rintf(v.x * inv), q1 = (int)rintf(v.y * inv), q2 = (int)rintf(v.z * inv),
              q3 = (int)rintf(v.w * inv);
    const uint32_t hi = ((uint32_t)(q0 >> 14) & 0xFFu) | (((uint32_t)(q1 >> 14) & 0xFFu) << 8) |
                        (((uint32_t)(q2 >> 14) & 0xFFu) << 16) | (((uint32_t)(q3 >> 14) & 0xFFu) << 24);
    const uint32_t mid = ((uint32_t)(q0 >> 7) & 0x7Fu) | (((uint32_t)(q1 >> 7) & 0x7Fu) << 8) |
                         (((uint32_t)(q2 >> 7) & 0x7Fu) << 16) | (((uint32_t)(q3 >> 7) & 0x7Fu) << 24);
    const uint32_t lo = ((uint32_t)q0 & 0x7Fu) | (((uint32_t)q1 & 0x7Fu) << 8) | (((uint32_t)q2 & 0x7Fu) << 16) |
                        (((uint32_t)q3 & 0x7Fu) << 24);
    const int C = c >> 2, wi = c & 3;
    hw[cslot(C) * 4 + wi] = hi;
    mw[cslot(C) * 4 + wi] = mid;
    lw[cslot(C) * 4 + wi] = lo;
    if ((c & 7) == 0) {
        xs[c >> 3] = amax / XQ_MAX;
        s32[c >> 3] = sum32;
    }
    if ((c & 3) == 0) s16[c >> 2] = sum16;
}

// One workgroup per CU of GW threads (GNW waves): the x prologue is done once
// per CU, and the waves of a CU take the row tiles of the workgroup's range
// from a counter in LDS, so waves that started late (their first loads queue
// behind the other waves') take fewer tiles and the CU finishes together.
constexpr int GW = 1024, GNW = GW / WAVE;

// x -> (optional RMSNorm, infer/ops.odin:7-19) -> 22-bit integers in LDS, in two
// phases so that the x loads are issued before the weight prefetch (vector
// loads return in order: x must not queue behind the weights).  XR float4 of
// x (and of the norm weight) per thread are held in registers; XR == 0 means
// K is too long for that and both passes read x from memory after the
// prefetch.  K/4 is a multiple of 8, so the 8-lane groups of quant4 are whole.
// Prologue modes: NORM 0 takes x as it is, XN_RMS replaces it by rmsnorm(x) *
// norm_w over the whole vector -- as norm_w * x, quantized without waiting
// for the sum of squares: the inverse RMS is one factor of the whole row, so
// xpre_finish returns it and the caller scales each row's dot product by it
// (one workgroup barrier instead of two); XN_GATED finishes the gated RMSNorm of a
// DeltaNet layer's output (qwen3_5/forward.odin:211-218): x holds o silu(z)
// per head of GN_HV values and gss the head's four partial sums of o^2;
// x = norm_w[j] (inv_h x), inv_h = 1 / sqrt(sum_h o^2 / GN_HV + eps).
// XN_RMS_CONV is XN_RMS with the conv epilogue (segment 0's rows are DeltaNet
// conv channels).
enum { XN_RMS = 1, XN_GATED = 2, XN_RMS_CONV = 3 };
constexpr int GN_HV = 128;
static constexpr bool xn_rms(int n) { return n == XN_RMS || n == XN_RMS_CONV; }

template <int XR, int NORM>
struct XPre {
    float4 x[XR > 0 ? XR : 1], w[XR > 0 && NORM ? XR : 1], z[XR > 0 && NORM == XN_GATED ? XR : 1];  // z: gss
};

template <int XR, int NORM, bool REV = false>
static __device__ __forceinline__ void xpre_load(const GemvArgs &a, XPre<XR, NORM> &p) {
    // unconditional loads (indices clamped to the last float4, duplicates are
    // ignored by xpre_finish): a branch-free sequence lets the compiler wait
    // for exactly these loads later, not for the weight loads issued after
    const int tid = threadIdx.x, last = a.K / 4 - 1;
    const float4 *gx = (const float4 *)a.x;
    const float4 *nw = (const float4 *)a.norm_w;
#pragma unroll
    for (int ii = 0; ii < XR; ii++) {
        const int i = REV ? XR - 1 - ii : ii;  // REV: same loads in another order (see gemv_q_kernel)
        const int c = min(tid + i * GW, last);
        p.x[i] = gx[c];
        if (xn_rms(NORM)) p.w[i] = nw[c];
        if (NORM == XN_GATED) {
            p.w[i] = nw[c % (GN_HV / 4)];
            p.z[i] = ((const float4 *)a.gss)[c / (GN_HV / 4)];
        }
    }
}

template <int XR, int NORM>
static __device__ __forceinline__ float xpre_finish(const GemvArgs &a, const XPre<XR, NORM> &p, u32x4 *xhi,
                                                    u32x4 *xmid, u32x4 *xlo, float *xs, float *s32, float *s16,
                                                    float *red) {
    static_assert(NORM != XN_GATED || XR > 0, "the gated norm needs x in registers");
    const int K = a.K, tid = threadIdx.x;
    const float4 *gx = (const float4 *)a.x;
    const float4 *nw = (const float4 *)a.norm_w;
    uint32_t *hw = (uint32_t *)xhi, *mw = (uint32_t *)xmid, *lw = (uint32_t *)xlo;
    if (NORM == XN_GATED) {
#pragma unroll
        for (int i = 0; i < XR; i++) {
            const float4 v = p.x[i], z = p.z[i], w = p.w[i];
            float4 g;
            {
#pragma clang fp contract(off)
                const float inv = 1.0f / sqrtf(((z.x + z.y) + (z.z + z.w)) / (float)GN_HV + a.eps);
                g.x = w.x * (inv * v.x);
                g.y = w.y * (inv * v.y);
                g.z = w.z * (inv * v.z);
                g.w = w.w * (inv * v.w);
            }
            const int c = tid + i * GW;
            if (c < K / 4) quant4(g, c, hw, mw, lw, xs, s32, s16);
        }
        __syncthreads();
        return 1.f;
    }
    auto one = [&](float4 v, float4 w, int c) {
        if (xn_rms(NORM)) {
#pragma clang fp contract(off)
            v.x = w.x * v.x;
            v.y = w.y * v.y;
            v.z = w.z * v.z;
            v.w = w.w * v.w;
        }
        quant4(v, c, hw, mw, lw, xs, s32, s16);
    };
    float ss = 0.f;
    if (XR > 0) {
#pragma unroll
        for (int i = 0; i < XR; i++) {
            const int c = tid + i * GW;
            if (c < K / 4) {
                const float4 v = p.x[i];
                if (xn_rms(NORM)) ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                one(v, p.w[NORM ? i : 0], c);
            }
        }
    } else {
        for (int c = tid; c < K / 4; c += GW) {
            const float4 v = gx[c];
            if (xn_rms(NORM)) ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            one(v, NORM ? nw[c] : v, c);
        }
    }
    if (xn_rms(NORM)) {
        ss = wave_sum(ss);
        if ((tid & (WAVE - 1)) == 0) red[tid / WAVE] = ss;
    }
    __syncthreads();
    if (!xn_rms(NORM)) return 1.f;
    // every thread sums the waves' partials in the same order
    float t[GNW / 2];
#pragma unroll
    for (int i = 0; i < GNW / 2; i++) t[i] = red[2 * i] + red[2 * i + 1];
#pragma unroll
    for (int w = GNW / 4; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; i++) t[i] = t[2 * i] + t[2 * i + 1];
    return 1.0f / sqrtf(t[0] / (float)K + a.eps);
}

// LDS of gemv_q_kernel: the x planes and scales, then the workgroup's outputs
static size_t gemv_q_lds(int K, int out_rows) {
    return (size_t)K / 16 * 48 + (size_t)K / 32 * 8 + (size_t)K / 16 * 4 + (size_t)out_rows * 4;
}

// One workgroup: row tiles [tb, te) of segment `seg`, all of weight type T.
// A tile is R rows per lane group x (64/lpr) groups: the rows one wave
// computes together, in upl = U/lpr steps of one unit per lane (one step
// when a row is at most 64 units long, XU1; then a lane's unit is the same
// in every step and its slice of x stays in registers).  A wave starts with
// tile `wave` and then takes the next free tile of the workgroup from the
// LDS counter.  The weights of a step are requested before the previous step
// is computed (two register stages); every pass issues the same loads (a
// step past the end reads row 0's first units, unused), so the compiler
// waits for exactly the stage it consumes.  Rows past the end of the matrix
// are clamped to the last row (computed, not stored).
template <int T, int R, int NM, int XR, bool XU1, int NORM, int MOE = 0>
static __device__ __forceinline__ void gemv_run(const GemvArgs &a, int seg, int tb, int te, int wg,
                                                const XPre<XR, NORM> &xp, int idv = 0, float wv = 0.f,
                                                float xsc_r = 1.f) {
    using W = typename Types<T>::W;
    using X = typename Types<T>::X;
    extern __shared__ u32x4 smem[];
    __shared__ float red[GNW];
    __shared__ int redi[GNW];
    __shared__ uint32_t tile_ctr;
    const int K = a.K, tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE;
    const DMat &m0 = a.seg[seg].m;
    const DMat &m1 = a.seg[NM == 2 ? 1 : seg].m;
    const int lpr = a.lpr, grp = lane / lpr, j = lane & (lpr - 1);
    // (MOE_COLS: lanes per row need not divide the units; a lane's units past
    // the row are read at the row's last unit and weighted 0)
    const int U = K >> 6, upl = XU1 ? 1 : (MOE == MOE_COLS ? (U + lpr - 1) / lpr : U / lpr);
    const int rows_m = m0.rows, rpt = a.rows_per_wg;
    const int ntl = te - tb;
    const int rsub = grp * R;

    W ring[2][NM][R];
    auto issue = [&](int t, int ui, W (&w)[NM][R]) {
        const bool live = t < ntl;
        const int u = XU1 ? j : j + ui * lpr;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = live ? min((tb + t) * rpt + rsub + r, rows_m - 1) : 0;
            int prow = row, pu = live ? (MOE == MOE_COLS ? min(u, U - 1) : u) : j;  // the stored row and unit
            if (MOE == MOE_ROWS || MOE == MOE_ROWS_R) {  // virtual row -> row of the chosen expert
                const int k = row / a.moe_blk;
                prow = __shfl(idv, k, WAVE) * a.moe_blk + (row - k * a.moe_blk);
            } else if (MOE == MOE_COLS) {  // unit of the concatenation -> unit of the chosen expert's row
                const int k = pu / a.moe_blk;
                prow = __shfl(idv, k, WAVE) * rows_m + row;
                pu -= k * a.moe_blk;
            }
            wload(m0, prow, pu, w[0][r]);
            if (NM == 2) wload(m1, prow, pu, w[NM - 1][r]);
        }
    };
    // x was requested by the caller; the first weights follow (loads return in order)
    int ct = wave, cu = 0;
    issue(ct, cu, ring[0]);
    __builtin_amdgcn_sched_barrier(0);
    // conv epilogue: this thread's row's taps and window (rows past the end
    // and other segments' workgroups read a valid row, unused), needed only
    // after the loop, so requested after the first weights (they come from
    // HBM; the weight requests do not wait for them)
    float ctap[4] = {0.f, 0.f, 0.f, 0.f}, cwin[3] = {0.f, 0.f, 0.f};
    if (NORM == XN_RMS_CONV) {
        const int KS = a.conv_kernel, km1 = KS - 1;
        const int c = min(tb * a.rows_per_wg + tid, a.seg[0].m.rows - 1);
#pragma unroll
        for (int k = 0; k < 4; k++) ctap[k] = a.conv_w[(size_t)c * KS + min(k, km1)];
#pragma unroll
        for (int k = 0; k < 3; k++) cwin[k] = a.conv_state[(size_t)c * km1 + min(k, km1 - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);

    u32x4 *xhi = smem, *xmid = smem + K / 16, *xlo = smem + 2 * (K / 16);
    float *xs = (float *)(smem + 3 * (K / 16)), *s32 = xs + K / 32, *s16 = s32 + K / 32;
    float *yo = s16 + K / 16;  // this workgroup's outputs
    const int wrow0 = tb * rpt, wrow1 = min(te * rpt, rows_m);
    if (tid == 0) tile_ctr = 0;  // read after the prologue's barriers
    // xsc: the RMSNorm's inverse RMS, a factor of every row's dot product
    float xsc = xsc_r;
    if (MOE == MOE_ROWS_R) __syncthreads();  // the kernel built the x planes before routing
    else xsc = xpre_finish<XR, NORM>(a, xp, xhi, xmid, xlo, xs, s32, s16, red);
    const XQ xq{xhi, xmid, xlo, xs, s32, s16};
    X xu;
    if (XU1) xload(xq, j, xu);

    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    float acc[NM][R];
#pragma unroll
    for (int i = 0; i < NM; i++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[i][r] = 0.f;

    // the step after (t, ui): the next unit of the tile, or the next free tile
    auto next = [&](int t, int ui, int &nt, int &nu) {
        if (ui + 1 < upl) {
            nt = t;
            nu = ui + 1;
        } else {
            uint32_t v = 0;
            if (lane == 0) v = __hip_atomic_fetch_add(&tile_ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            nt = GNW + (int)__builtin_amdgcn_readfirstlane(v);
            nu = 0;
        }
    };
    auto compute = [&](int t, int ui, const W (&w)[NM][R]) {
        const int u0 = XU1 ? j : j + ui * lpr;
        const int u = MOE == MOE_COLS ? min(u0, U - 1) : u0;
        if (!XU1) xload(xq, u, xu);
        // (MOE_COLS: the unit's expert weight; units keep their position in the
        // super-block, as each expert's part is a whole number of super-blocks)
        const float uw0 = MOE == MOE_COLS ? __shfl(wv, u / a.moe_blk, WAVE) : 1.f;
        const float uw = MOE == MOE_COLS && u0 >= U ? 0.f : uw0;
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (MOE == MOE_COLS) acc[0][r] += uw * wdot(w[0][r], u, xu);
            else acc[0][r] += wdot(w[0][r], u, xu);
            if (NM == 2) acc[NM - 1][r] += wdot(w[NM - 1][r], u, xu);
        }
        if (XU1 || ui == upl - 1) {
            // reduce over the lanes of the row; results go to LDS (no global
            // memory traffic in the loop but the weight loads)
#pragma unroll
            for (int r = 0; r < R; r++) {
                acc[0][r] = lane_group_sum(acc[0][r], lpr);
                if (NM == 2) acc[NM - 1][r] = lane_group_sum(acc[NM - 1][r], lpr);
            }
            if (j == 0) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int row = (tb + t) * rpt + rsub + r;
                    float val = acc[0][r] * xsc;
                    if (NM == 2) {  // infer/forward.odin:128-132
#pragma clang fp contract(off)
                        val *= 1.0f / (1.0f + expf(-val));
                        val *= acc[NM - 1][r] * xsc;
                    }
                    yo[row - wrow0] = val;  // rows past the matrix land in the slack of yo
                    if (NM == 1 && a.mode == GEMV_ARGMAX && row < rows_m && better(val, row, bv, bi)) {
                        bv = val;
                        bi = row;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < NM; i++)
#pragma unroll
                for (int r = 0; r < R; r++) acc[i][r] = 0.f;
        }
    };
    // two steps per pass, so the ring stage of each step is static
    while (ct < ntl) {
        int nt, nu;
        next(ct, cu, nt, nu);
        issue(nt, nu, ring[1]);
        __builtin_amdgcn_sched_barrier(0);  // the loads go out before this step's arithmetic
        compute(ct, cu, ring[0]);
        ct = nt;
        cu = nu;
        if (ct >= ntl) break;
        next(ct, cu, nt, nu);
        issue(nt, nu, ring[0]);
        __builtin_amdgcn_sched_barrier(0);
        compute(ct, cu, ring[1]);
        ct = nt;
        cu = nu;
    }

    // write back the workgroup's contiguous rows (coalesced)
    __syncthreads();
    {
        float *y = a.seg[seg].y;
        // shared-expert gate: y += sigmoid(g) * Wx (the product first, then the scale)
        const float gs = NM == 1 && a.mode == GEMV_ADD && a.ygate ? 1.0f / (1.0f + expf(-a.ygate[0])) : 1.f;
        if (NORM == XN_RMS_CONV && seg == 0) {
            // conv epilogue: row c is a channel of the DeltaNet conv
            // (qwen3_5/ops.odin:97-116, as dn_conv_kernel): silu of the window with the
            // product last, then the window slides (2 <= kernel <= 4)
            const int KS = a.conv_kernel, km1 = KS - 1;
            for (int i = tid; i < wrow1 - wrow0; i += GW) {
#pragma clang fp contract(off)
                const int c = wrow0 + i;
                float *cs = a.conv_state + (size_t)c * km1;
                float tp[4], wn[3];
#pragma unroll
                for (int k = 0; k < 4; k++) tp[k] = i == tid ? ctap[k] : a.conv_w[(size_t)c * KS + min(k, km1)];
#pragma unroll
                for (int k = 0; k < 3; k++) wn[k] = i == tid ? cwin[k] : cs[min(k, km1 - 1)];
                const float x = yo[i];
                float acc = tp[km1] * x;
#pragma unroll
                for (int k = 0; k < 3; k++)
                    if (k < km1) acc += tp[k] * wn[k];
                y[c] = silu_ref(acc);
#pragma unroll
                for (int k = 0; k < 2; k++)
                    if (k < km1 - 1) cs[k] = wn[k + 1];
                cs[km1 - 1] = x;
            }
        } else {
            for (int i = tid; i < wrow1 - wrow0; i += GW) {
                if (NM == 1 && a.mode == GEMV_ADD) y[wrow0 + i] = y[wrow0 + i] + (a.ygate ? yo[i] * gs : yo[i]);
                else y[wrow0 + i] = yo[i];
            }
        }
    }
    if (NM == 1 && a.mode == GEMV_ARGMAX) {  // this workgroup's best (value, lowest row)
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, WAVE);
            const int oi = __shfl_xor(bi, o, WAVE);
            if (better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            red[wave] = bv;
            redi[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < GNW; w++)
                if (better(red[w], redi[w], bv, bi)) {
                    bv = red[w];
                    bi = redi[w];
                }
            a.am_val[wg] = bv;
            a.am_idx[wg] = bi;
            if (wg == 0) a.state[ST_PENDING] = 1;  // argmax pending for the next embedding step
        }
    }
}

// lane j's value, broadcast to the wave (j uniform)
static __device__ __forceinline__ float readlanef(float v, int j) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// number of set bits of m below this lane
static __device__ __forceinline__ int lane_prefix(unsigned long long m) {
    return (int)__builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
}

// Wave max and sum without LDS: DPP within rows of 16 lanes, then the four
// rows' results read out of lanes 0, 16, 32, 48 (sum: ((r0 + r1) + r2) + r3,
// the same on every lane).
static __device__ __forceinline__ float wave_max_dpp(float v) {
    v = dpp_max8(v);
    v = fmaxf(v, OI_DPP(v, 0x140));
    return fmaxf(fmaxf(readlanef(v, 0), readlanef(v, 16)), fmaxf(readlanef(v, 32), readlanef(v, 48)));
}
static __device__ __forceinline__ float wave_sum_dpp(float v) {
    v = lane_group_sum(v, 16);
    return ((readlanef(v, 0) + readlanef(v, 16)) + readlanef(v, 32)) + readlanef(v, 48);
}

// Expert keys for routing: bit 41 set for a defined probability p (>= +0,
// so its bits order as unsigned integers), p's bits at 40..10, 1023 - id at
// 9..0: one unsigned comparison orders experts by (p descending, id
// ascending); an undefined expert (NaN p, or past n) has key 0.
constexpr unsigned long long ROUTE_KEY_VALID = 1ull << 41;
static_assert(GW <= 1024, "expert ids must fit the key's 10 low bits");


// Routing of one token inside the workgroup (MoE rows mode): the router
// logits l[0..n) (n <= GW) -> softmax (max, exp(l - max), sum, divide: the
// oracle's ref_softmax) -> the k best experts in the order (p descending, id
// ascending), i.e. the order of k rounds of first-maximum selection -> lane
// r < moe_k of every wave gets the id of rank r and its weight (p, or p / the
// sum of the chosen in rank order).  Workgroup
// 0 also writes them out for the down projection and the caller.  The loads
// were issued by the caller before the weights'.
static __device__ __forceinline__ void moe_route(const GemvArgs &a, float lg, float sg, int &idv, float &wv, int wg) {
    __shared__ float rmax[GNW], rsum[GNW];
    __shared__ unsigned long long cand[GW];     // wave w's best keys at [w * k, w * k + k), then zeros
    __shared__ unsigned long long stage[WAVE];  // keys moved between the lanes of wave 0
    __shared__ unsigned long long ordered[WAVE];  // the chosen keys by rank
    __shared__ int rid[WAVE];                   // the chosen ids and weights, rank order
    __shared__ float rw[WAVE];
    const int n = a.moe_n, t = threadIdx.x, lane = t & (WAVE - 1), wave = t / WAVE;
    const int k = a.moe_sel > 0 ? a.moe_sel : a.moe_k, nw = (n + WAVE - 1) / WAVE;
    const float m = wave_max_dpp(t < n ? lg : -INFINITY);
    if (lane == 0) rmax[wave] = m;
    __syncthreads();
    float M = rmax[0];
#pragma unroll
    for (int w = 1; w < GNW; w++) M = fmaxf(M, rmax[w]);
    float e = 0.f;
    if (t < n) {
#pragma clang fp contract(off)
        e = expf(lg - M);
    }
    const float es = wave_sum_dpp(e);
    if (lane == 0) rsum[wave] = es;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < GNW; w++) tot += rsum[w];
    const float pi = e / tot;
    // Two levels: each wave's k best of its 64 experts become candidates (an
    // expert among the k best overall has fewer than k better experts in its
    // wave); then wave 0 takes the k best candidates (every expert better
    // than one of the k best overall is itself a candidate) and orders them.
    // The bit searches run on the CU's one scalar unit, so the second level
    // is not repeated in every wave.  A rank no expert fills keeps id 0,
    // weight 0.
    const bool valid = t < n && pi == pi;
    const unsigned long long key =
        valid ? ROUTE_KEY_VALID | ((unsigned long long)__float_as_uint(pi) << 10) | (unsigned)(1023 - t) : 0ull;
    if (wave < nw) {
        const unsigned long long v[1] = {key};
        const unsigned long long T = __popcll(__ballot(valid)) > k ? wave_kth_key(v, k) : 0ull;
        const bool c = valid && key >= T;
        const unsigned long long cm = __ballot(c);
        if (c) cand[wave * k + lane_prefix(cm)] = key;
        if (lane >= __popcll(cm) && lane < k) cand[wave * k + lane] = 0ull;
    }
    __syncthreads();
    if (wave == 0) {
        // the candidates, 64 at a time: lanes < k of A keep the best so far
        const int nc = nw * k;
        unsigned long long A = lane < nc ? cand[lane] : 0ull;
        for (int c0 = WAVE; c0 < nc; c0 += WAVE) {
            const unsigned long long v[2] = {A, c0 + lane < nc ? cand[c0 + lane] : 0ull};
            const int nv = __popcll(__ballot(v[0] != 0ull)) + __popcll(__ballot(v[1] != 0ull));
            const unsigned long long T = nv > k ? wave_kth_key(v, k) : 0ull;
            const bool w0 = v[0] != 0ull && v[0] >= T, w1 = v[1] != 0ull && v[1] >= T;
            const unsigned long long b0 = __ballot(w0), b1 = __ballot(w1);
            if (w0) stage[lane_prefix(b0)] = v[0];
            if (w1) stage[__popcll(b0) + lane_prefix(b1)] = v[1];
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
            __builtin_amdgcn_wave_barrier();
            A = lane < __popcll(b0) + __popcll(b1) ? stage[lane] : 0ull;
            __builtin_amdgcn_wave_barrier();
        }
        // the k best, ordered: lane r gets the key of rank r (0 past the last);
        // the chosen keys are read back from LDS by every lane (broadcast
        // reads, all in flight together)
        const unsigned long long v[1] = {A};
        const unsigned long long T = __popcll(__ballot(A != 0ull)) > k ? wave_kth_key(v, k) : 0ull;
        const bool win = A != 0ull && A >= T;
        const unsigned long long bw = __ballot(win);
        const int nch = __popcll(bw);
        if (win) stage[lane_prefix(bw)] = A;
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        const unsigned long long mine = lane < nch ? stage[lane] : 0ull;
        int rank = 0;
        for (int j = 0; j < nch; j++) rank += stage[j] > mine ? 1 : 0;
        if (lane < nch) ordered[rank] = mine;
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        const unsigned long long R = lane < nch ? ordered[lane] : 0ull;
        const float wr = R != 0ull ? __uint_as_float((unsigned)(R >> 10) & 0x7FFFFFFFu) : 0.f;
        const int id = R != 0ull ? 1023 - (int)(R & 1023u) : 0;
        float s = 0.f;  // in rank order, as the sequential selection; ranks past nch weigh 0
        for (int r = 0; r < nch; r++) s += __uint_as_float((unsigned)(ordered[r] >> 10) & 0x7FFFFFFFu);
        const int nblk = a.moe_nblk > 0 ? a.moe_nblk : n;
        if (lane < a.moe_k) {
            int fi;
            float fw;
            if (lane < k) {
                fi = min(max(id, 0), nblk - 1);
                fw = a.moe_norm ? wr / s : wr;
            } else {  // the shared expert, gated by sigmoid of its router row
                fi = n;
                fw = 1.0f / (1.0f + expf(-sg));
            }
            rid[lane] = fi;
            rw[lane] = fw;
            if (wg == 0) {
                a.moe_ids_out[lane] = fi;
                a.moe_w_out[lane] = fw;
            }
        }
    }
    __syncthreads();
    if (lane < a.moe_k) {
        idv = rid[lane];
        wv = rw[lane];
    }
}

// Router of a routed-expert layer fused into the gate/up launch (MOE_ROWS_R):
// l[r] = router row r . x for r < moe_n, from the x planes in LDS -- the
// router GEMV's arithmetic (the same 64-weight units, int8 products, per-unit
// scaling), lanes per row = K / 64 (32 or 64).  The rows of up to RR steps
// are requested at the kernel's start, before the x prologue (a workgroup
// reads the router from L2, the first of each XCD from HBM), and consumed
// after it; longer routers take further passes.
template <int T>
struct RouterPre {
    static constexpr int RR = T == T_Q4_K ? 4 : 2;  // (a Q6_K / Q8_0 unit holds more registers)
    typename Types<T>::W w[RR];
};
// (the waves' rows are rotated by the workgroup index, so the workgroups of
// an XCD do not request the same router rows at the same moment)
template <int T>
static __device__ __forceinline__ void router_row(const GemvArgs &a, int base, int st, int &r, int &j) {
    const int U = a.K >> 6, lane = threadIdx.x & (WAVE - 1), rpw = WAVE / U;
    const int wave = ((int)(threadIdx.x / WAVE) + (int)blockIdx.x) & (GNW - 1);
    j = lane & (U - 1);
    r = base + (st * GNW + wave) * rpw + lane / U;
}
template <int T>
static __device__ __forceinline__ void router_load(const GemvArgs &a, int base, RouterPre<T> &p) {
#pragma unroll
    for (int st = 0; st < RouterPre<T>::RR; st++) {
        int r, j;
        router_row<T>(a, base, st, r, j);
        wload(a.moe_router, min(r, a.moe_n - 1), j, p.w[st]);
    }
}
template <int T>
static __device__ __forceinline__ void router_logits(const GemvArgs &a, const XQ &xq, RouterPre<T> &p, float *rl,
                                                     float xsc) {
    using X = typename Types<T>::X;
    constexpr int RR = RouterPre<T>::RR;
    const int U = a.K >> 6, rpw = WAVE / U, n = a.moe_n;
    int r, j;
    router_row<T>(a, 0, 0, r, j);
    X xu;
    xload(xq, j, xu);
    for (int base = 0; base < n; base += GNW * rpw * RR) {
        if (base > 0) router_load<T>(a, base, p);
#pragma unroll
        for (int st = 0; st < RR; st++) {
            const float v = lane_group_sum(wdot(p.w[st], j, xu), U) * xsc;
            router_row<T>(a, base, st, r, j);
            if (j == 0 && r < n) rl[r] = v;
        }
    }
}

// Weight types are template parameters: T for every segment but the last,
// TL for the last (TL == T: one type).  A runtime switch over all types would
// let the compiler merge the code paths, and at the merge it can no longer
// count the loads in flight, so it waits for all of them; the two arms here
// issue their x loads in different orders so that they are not merged.
// Every wave waits for its x loads before it requests weights: x was written
// by the previous kernel and is read from the shared cache level, where it
// would otherwise queue behind the other CUs' weight requests (the prologue
// then ends later than the first weights arrive).  Other
// type mixes are issued as one launch per type (wg_base).
template <int T, int TL, int R, int NM, int XR, bool XU1, int NORM, int MOE = 0>
__global__ __launch_bounds__(GW) void gemv_q_kernel(GemvArgs a) {
    const int wg = blockIdx.x + a.wg_base;
    int seg = 0;
    if (NM == 1)
        for (int i = 1; i < a.nseg; i++)
            if (wg >= a.seg[i].wg_begin) seg = i;
    const int seg_end = (NM == 1 && seg + 1 < a.nseg) ? a.seg[seg + 1].wg_begin : a.total_wgs;
    const int nwg = seg_end - a.seg[seg].wg_begin, w = wg - a.seg[seg].wg_begin;
    const int ntiles = a.seg[seg].ntiles;
    const int tb = (int)((long)ntiles * w / nwg), te = (int)((long)ntiles * (w + 1) / nwg);
    if (TL != T && seg == a.nseg - 1) {
        XPre<XR, NORM> xp;
        xpre_load<XR, NORM, true>(a, xp);  // x first, then the weights (loads return in order)
        __builtin_amdgcn_sched_barrier(0);  // keep every x load ahead of the weight loads
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __builtin_amdgcn_sched_barrier(0);
        gemv_run<TL, R, NM, XR, XU1, NORM>(a, seg, tb, te, wg, xp);
    } else if (MOE == MOE_ROWS_R) {
        // the x prologue here (RMSNorm, the quantized planes in LDS, as
        // gemv_run's), the router logits from it, the routing, then the
        // chosen experts' rows
        XPre<XR, NORM> xp;
        xpre_load<XR, NORM>(a, xp);
        __builtin_amdgcn_sched_barrier(0);  // x first: the router rows queue behind it, not before
        RouterPre<T> rp;
        router_load<T>(a, 0, rp);
        __builtin_amdgcn_sched_barrier(0);
        extern __shared__ u32x4 smem[];
        __shared__ float red_r[GNW], rl[GW];
        const int K = a.K;
        u32x4 *xhi = smem, *xmid = smem + K / 16, *xlo = smem + 2 * (K / 16);
        float *xs = (float *)(smem + 3 * (K / 16)), *s32 = xs + K / 32, *s16 = s32 + K / 32;
        const float xsc = xpre_finish<XR, NORM>(a, xp, xhi, xmid, xlo, xs, s32, s16, red_r);
        const XQ xq{xhi, xmid, xlo, xs, s32, s16};
        router_logits<T>(a, xq, rp, rl, xsc);
        __syncthreads();
        int idv = 0;
        float wv = 0.f;
        moe_route(a, (int)threadIdx.x < a.moe_n ? rl[threadIdx.x] : 0.f, 0.f, idv, wv, wg);
        gemv_run<T, R, NM, XR, XU1, NORM, MOE>(a, seg, tb, te, wg, xp, idv, wv, xsc);
    } else {
        XPre<XR, NORM> xp;
        xpre_load<XR, NORM>(a, xp);
        // routed experts: lane l < moe_k holds expert l's id (and weight)
        int idv = 0;
        float wv = 0.f;
        float lg = 0.f, sg = 0.f;
        const bool route = MOE == MOE_ROWS && a.moe_logits != nullptr;
        if (MOE) {
            const int l = threadIdx.x & (WAVE - 1);
            if (route) {
                if ((int)threadIdx.x < a.moe_n) lg = a.moe_logits[threadIdx.x];
                if (a.moe_sgate) sg = a.moe_sgate[0];
            } else if (l < a.moe_k) {
                // ids come from the device
                idv = min(max(a.moe_ids[l], 0), (a.moe_nblk > 0 ? a.moe_nblk : a.moe_n) - 1);
                if (MOE == MOE_COLS) wv = a.moe_w[l];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): x has arrived before any weight request goes out
        __builtin_amdgcn_sched_barrier(0);
        if (route) moe_route(a, lg, sg, idv, wv, wg);
        gemv_run<T, R, NM, XR, XU1, NORM, MOE>(a, seg, tb, te, wg, xp, idv, wv);
    }
}

// kernel configurations: (R, NM, XR, XU1); XR = float4 of x per thread held
// in registers by the prologue (K <= 4 * GW * XR), 0 = x read twice from
// memory; XU1 = one unit per lane per row (K <= 4096), x kept in registers
template <int T, int R, int NORM>
static const void *gemv_q_fn_r(bool swiglu, bool xu1, int K) {
    if constexpr (NORM == XN_GATED || NORM == XN_RMS_CONV) {  // x in registers: K <= 4096
        if (swiglu || K > 4096 || (NORM == XN_GATED && K % GN_HV)) return nullptr;
        if (xu1) return (const void *)gemv_q_kernel<T, T, R, 1, 1, true, NORM>;
        return (const void *)gemv_q_kernel<T, T, R, 1, 1, false, NORM>;
    } else {
        if (swiglu) {
            if (K <= 4096 && xu1) return (const void *)gemv_q_kernel<T, T, 1, 2, 1, true, NORM>;
            if (K <= 4096) return (const void *)gemv_q_kernel<T, T, 1, 2, 1, false, NORM>;
            return (const void *)gemv_q_kernel<T, T, 1, 2, 0, false, NORM>;
        }
        if (K <= 4096 && xu1) return (const void *)gemv_q_kernel<T, T, R, 1, 1, true, NORM>;
        if (K <= 4096) return (const void *)gemv_q_kernel<T, T, R, 1, 1, false, NORM>;
        if (K <= 12288) return (const void *)gemv_q_kernel<T, T, R, 1, 3, false, NORM>;
        return (const void *)gemv_q_kernel<T, T, R, 1, 0, false, NORM>;
    }
}
template <int T, int NORM>
static const void *gemv_q_fn_t(bool swiglu, bool xu1, int K, int R) {
    return R == 1 ? gemv_q_fn_r<T, 1, NORM>(swiglu, xu1, K) : nullptr;
}
// two-type kernels (first segments T, last segment TL; RMSNorm prologue,
// K <= 4096): the projection GEMVs of a layer
template <int T, int TL>
static const void *gemv_q_fn_mixed(bool xu1, int K, int R) {
    if (K > 4096 || R != 1) return nullptr;
    if (xu1) return (const void *)gemv_q_kernel<T, TL, 1, 1, 1, true, true>;
    return (const void *)gemv_q_kernel<T, TL, 1, 1, 1, false, true>;
}
static bool xu1_of(int K) {
    const int U = K / 64;
    return U <= 64 && (U & (U - 1)) == 0;  // one unit per lane per row
}
static const void *gemv_q_fn_mixed(int t, int tl, int norm, int K, int R) {
    const bool xu1 = xu1_of(K);
    if (norm != XN_RMS) return nullptr;
    if (t == T_Q4_K && tl == T_Q6_K) return gemv_q_fn_mixed<T_Q4_K, T_Q6_K>(xu1, K, R);
    if (t == T_Q6_K && tl == T_Q4_K) return gemv_q_fn_mixed<T_Q6_K, T_Q4_K>(xu1, K, R);
    if (t == T_Q4_K && tl == T_Q8_0) return gemv_q_fn_mixed<T_Q4_K, T_Q8_0>(xu1, K, R);
    if (t == T_Q8_0 && tl == T_Q4_K) return gemv_q_fn_mixed<T_Q8_0, T_Q4_K>(xu1, K, R);
    if (t == T_Q8_0 && tl == T_Q6_K) return gemv_q_fn_mixed<T_Q8_0, T_Q6_K>(xu1, K, R);
    if (t == T_Q6_K && tl == T_Q8_0) return gemv_q_fn_mixed<T_Q6_K, T_Q8_0>(xu1, K, R);
    return nullptr;
}
template <int T>
static const void *gemv_q_fn_n(bool swiglu, int norm, bool xu1, int K, int R) {
    if (norm == XN_GATED) return gemv_q_fn_t<T, XN_GATED>(swiglu, xu1, K, R);
    if (norm == XN_RMS_CONV) return gemv_q_fn_t<T, XN_RMS_CONV>(swiglu, xu1, K, R);
    return norm ? gemv_q_fn_t<T, XN_RMS>(swiglu, xu1, K, R) : gemv_q_fn_t<T, 0>(swiglu, xu1, K, R);
}
static const void *gemv_q_fn(int type, bool swiglu, int norm, int K, int R) {
    const bool xu1 = xu1_of(K);
    switch (type) {
    case T_Q4_K: return gemv_q_fn_n<T_Q4_K>(swiglu, norm, xu1, K, R);
    case T_Q6_K: return gemv_q_fn_n<T_Q6_K>(swiglu, norm, xu1, K, R);
    default: return gemv_q_fn_n<T_Q8_0>(swiglu, norm, xu1, K, R);
    }
}
// the prologue mode of a GEMV's arguments
static int norm_mode(const GemvArgs &a) {
    return a.gss ? XN_GATED : a.norm_w ? (a.conv_w ? XN_RMS_CONV : XN_RMS) : 0;
}


// rows per lane group of a plan (the kernel's R)
static int plan_r(const GemvArgs &a) { return a.rows_per_wg / (64 / a.lpr); }

// One launch when the segments are of one type, or of one type but the
// last; otherwise one launch per run of consecutive segments of one type.
static const void *gemv_q_fn_all(const GemvArgs &a) {
    if (a.mode == GEMV_SWIGLU || a.nseg < 2) return nullptr;
    for (int i = 1; i < a.nseg - 1; i++)
        if (a.seg[i].m.type != a.seg[0].m.type) return nullptr;
    const int t = a.seg[0].m.type, tl = a.seg[a.nseg - 1].m.type;
    if (tl == t) return gemv_q_fn(t, false, norm_mode(a), a.K, plan_r(a));
    return gemv_q_fn_mixed(t, tl, norm_mode(a), a.K, plan_r(a));
}

bool gemv_q_supported(const GemvArgs &a) {
    const int n = a.mode == GEMV_SWIGLU ? 2 : a.nseg;
    for (int i = 0; i < n; i++) {
        const int t = a.seg[i].m.type;
        if (t != T_Q4_K && t != T_Q6_K && t != T_Q8_0) return false;
    }
    if (a.mode == GEMV_SWIGLU && a.seg[0].m.type != a.seg[1].m.type) return false;
    // the x prologue holds K/16 chunks of three planes in LDS
    if (gemv_q_lds(a.K, 0) > 96 * 1024) return false;
    // gated head norm prologue: x in registers, whole heads; conv epilogue: stored rows
    if (a.gss && (!a.norm_w || a.mode == GEMV_SWIGLU || a.K > 4096 || a.K % GN_HV)) return false;
    if (a.conv_w && (a.mode != GEMV_STORE || !a.norm_w || !a.conv_state || a.conv_kernel < 2 ||
                     a.conv_kernel > 4 || a.K > 4096))
        return false;
    return a.K % 256 == 0 || (a.K % 64 == 0 && a.seg[0].m.type == T_Q8_0 && n == 1);
}

static int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

static double weight_bytes(int type) { return type == T_Q4_K ? 0.5625 : type == T_Q6_K ? 0.8203125 : 1.0625; }

// Plan for gemv_q_kernel: one workgroup per CU.  A tile is the rows of one
// wave (64/lpr lane groups x R rows).  Workgroups go to the segments in
// proportion to their bytes, each with a contiguous range of tiles of one
// segment.
void plan_gemv_q(GemvArgs &a) {
    const int U = a.K / 64;
    int lpr = 1;
    while (lpr < 64 && U % (lpr * 2) == 0) lpr *= 2;
    // routed-expert columns mode masks the units past the row, so a long row
    // takes a whole wave (one row per tile) whatever its unit count
    if (a.moe_ids && !a.moe_logits && a.mode != GEMV_SWIGLU && U >= 64) lpr = 64;
    a.lpr = lpr;
    const bool sw = a.mode == GEMV_SWIGLU;
    const int gpw = 64 / lpr, G = device_cus();
    const int nseg = sw ? 1 : a.nseg;
    long rows = 0;
    for (int i = 0; i < nseg; i++) rows += a.seg[i].m.rows;
    // (R = 2 measured no faster and does not fit 128 registers for every type)
    const int R = 1;
    (void)rows;
    a.rows_per_wg = gpw * R;
    double bytes[GEMV_MAX_SEG], total = 0;
    long total_tiles = 0;
    for (int i = 0; i < nseg; i++) {
        a.seg[i].ntiles = (a.seg[i].m.rows + a.rows_per_wg - 1) / a.rows_per_wg;
        total_tiles += a.seg[i].ntiles;
        bytes[i] = (double)a.seg[i].m.rows * a.K * weight_bytes(a.seg[i].m.type);
        total += bytes[i];
    }
    // at least one workgroup per segment; small matrices spread over more CUs
    // (4 tiles per workgroup) rather than filling every wave of a few
    const int nwg = (int)std::max<long>(nseg, std::min<long>(G, (total_tiles + 3) / 4));
    int wg = 0, left = nwg;
    for (int i = 0; i < nseg; i++) {
        a.seg[i].wg_begin = wg;
        int n = i == nseg - 1 ? left : (int)std::lround(nwg * bytes[i] / total);
        n = std::max(1, std::min(n, left - (nseg - 1 - i)));
        wg += n;
        left -= n;
    }
    if (sw) {
        a.seg[1].wg_begin = 0;
        a.seg[1].ntiles = a.seg[0].ntiles;
    }
    a.total_wgs = wg;
    int most = 0;
    for (int i = 0; i < nseg; i++) {
        const int end = i + 1 < nseg ? a.seg[i + 1].wg_begin : wg;
        const int n = end - a.seg[i].wg_begin;
        most = std::max(most, (a.seg[i].ntiles + n - 1) / n);
    }
    a.tiles_per_wg = most;
    a.kernel = 1;
}

// routed experts: one weight type; MOE_ROWS is the SwiGLU pair (optionally
// with the RMSNorm prologue), MOE_COLS a single matrix whose experts' parts
// are whole super-blocks (store or residual add)
template <int T, int MOE>
static const void *gemv_q_moe_fn(int K, bool norm) {
    const bool xu1 = xu1_of(K);
    if (MOE == MOE_ROWS) {
        if (K > 4096) return nullptr;
        if (norm) {
            if (xu1) return (const void *)gemv_q_kernel<T, T, 1, 2, 1, true, true, MOE_ROWS>;
            return (const void *)gemv_q_kernel<T, T, 1, 2, 1, false, true, MOE_ROWS>;
        }
        if (xu1) return (const void *)gemv_q_kernel<T, T, 1, 2, 1, true, false, MOE_ROWS>;
        return (const void *)gemv_q_kernel<T, T, 1, 2, 1, false, false, MOE_ROWS>;
    }
    if (MOE == MOE_ROWS_R) {  // the router needs RMSNorm(x): norm only
        if ((K != 2048 && K != 4096) || !norm) return nullptr;
        if (xu1) return (const void *)gemv_q_kernel<T, T, 1, 2, 1, true, true, MOE_ROWS_R>;
        return (const void *)gemv_q_kernel<T, T, 1, 2, 1, false, true, MOE_ROWS_R>;
    }
    if (norm) return nullptr;
    if (K <= 4096 && xu1) return (const void *)gemv_q_kernel<T, T, 1, 1, 1, true, false, MOE_COLS>;
    if (K <= 4096) return (const void *)gemv_q_kernel<T, T, 1, 1, 1, false, false, MOE_COLS>;
    if (K <= 12288) return (const void *)gemv_q_kernel<T, T, 1, 1, 3, false, false, MOE_COLS>;
    return nullptr;
}
template <int T>
static const void *gemv_q_moe_fn_t(int moe, int K, bool norm) {
    switch (moe) {
    case MOE_ROWS: return gemv_q_moe_fn<T, MOE_ROWS>(K, norm);
    case MOE_ROWS_R: return gemv_q_moe_fn<T, MOE_ROWS_R>(K, norm);
    case MOE_COLS: return gemv_q_moe_fn<T, MOE_COLS>(K, norm);
    default: return nullptr;
    }
}
static const void *gemv_q_moe_fn(int type, int moe, int K, bool norm) {
    switch (type) {
    case T_Q4_K: return gemv_q_moe_fn_t<T_Q4_K>(moe, K, norm);
    case T_Q6_K: return gemv_q_moe_fn_t<T_Q6_K>(moe, K, norm);
    case T_Q8_0: return gemv_q_moe_fn_t<T_Q8_0>(moe, K, norm);
    default: return nullptr;
    }
}

bool gemv_q_moe_supported(const GemvArgs &a, int moe) {
    if ((a.norm_w && moe != MOE_ROWS && moe != MOE_ROWS_R) || a.gss || a.conv_w || a.moe_k < 1 ||
        a.moe_k > WAVE || a.moe_n < 1 || a.moe_blk < 1)
        return false;
    if (moe == MOE_ROWS) {
        if (a.mode != GEMV_SWIGLU || a.seg[0].m.rows != a.moe_k * a.moe_blk) return false;
        const int sel = a.moe_sel > 0 ? a.moe_sel : a.moe_k;
        if (a.moe_sel > 0 && (a.moe_sel + 1 != a.moe_k || !a.moe_sgate || a.moe_nblk != a.moe_n + 1)) return false;
        if (a.moe_logits ? (a.moe_n > GW || sel > a.moe_n || !a.moe_ids_out || !a.moe_w_out) : !a.moe_ids)
            return false;
    } else if (moe == MOE_ROWS_R) {
        // no shared expert; the router in the experts' type, one row per expert
        if (a.mode != GEMV_SWIGLU || a.seg[0].m.rows != a.moe_k * a.moe_blk || a.moe_sel > 0 || !a.norm_w ||
            a.moe_n > GW || a.moe_k > a.moe_n || !a.moe_ids_out || !a.moe_w_out || a.moe_router.rows != a.moe_n ||
            a.moe_router.cols != a.K || a.moe_router.type != a.seg[0].m.type || !a.moe_router.q)
            return false;
    } else if (moe == MOE_COLS) {
        if ((a.mode != GEMV_STORE && a.mode != GEMV_ADD) || a.nseg != 1 || !a.moe_ids || !a.moe_w || a.moe_blk % 4 ||
            a.K != a.moe_k * 64 * a.moe_blk ||
            a.seg[0].m.cols != 64 * a.moe_blk)
            return false;
    } else {
        return false;
    }
    return gemv_q_supported(a) && gemv_q_moe_fn(a.seg[0].m.type, moe, a.K, a.norm_w != nullptr) != nullptr;
}

hipError_t launch_gemv_q_moe(const GemvArgs &a, int moe, hipStream_t st) {
    const void *fn = gemv_q_moe_supported(a, moe) ? gemv_q_moe_fn(a.seg[0].m.type, moe, a.K, a.norm_w != nullptr)
                                                   : nullptr;
    if (!fn) return hipErrorInvalidValue;
    GemvArgs b = a;
    b.wg_base = 0;
    void *args[] = {(void *)&b};
    const size_t lds = gemv_q_lds(a.K, a.tiles_per_wg * a.rows_per_wg);
    return hipLaunchKernel(fn, dim3(a.total_wgs), dim3(GW), args, lds, st);
}

hipError_t launch_gemv_q(const GemvArgs &a, hipStream_t st) {
    const bool sw = a.mode == GEMV_SWIGLU;
    const int nseg = sw ? 1 : a.nseg;
    const size_t lds = gemv_q_lds(a.K, a.tiles_per_wg * a.rows_per_wg);
    const int R = plan_r(a);
    if (const void *fn = gemv_q_fn_all(a)) {
        GemvArgs b = a;
        b.wg_base = 0;
        void *args[] = {(void *)&b};
        return hipLaunchKernel(fn, dim3(a.total_wgs), dim3(GW), args, lds, st);
    }
    for (int i = 0; i < nseg;) {
        int j = i + 1;
        while (j < nseg && a.seg[j].m.type == a.seg[i].m.type) j++;
        GemvArgs b = a;
        b.wg_base = a.seg[i].wg_begin;
        const int end = j < nseg ? a.seg[j].wg_begin : a.total_wgs;
        const void *fn = gemv_q_fn(a.seg[i].m.type, sw, norm_mode(a), a.K, R);
        if (!fn) return hipErrorInvalidValue;
        void *args[] = {(void *)&b};
        const hipError_t e = hipLaunchKernel(fn, dim3(end - b.wg_base), dim3(GW), args, lds, st);
        if (e != hipSuccess) return e;
        i = j;
    }
    return hipSuccess;
}

// ------------------------------------ routed experts of a short prefill chunk
// mt_dot4_kernel: the token loop's int8 dot4 arithmetic over the few pairs
// (<= MT_MFMA_FEW) of one expert slice.  An item is (expert, pair slice, one
// matrix); its workgroup (4 waves) streams every row of that matrix.  The
// prologue quantizes each pair's x row (silu(x) * x2 when x2 is set) into the
// three int8 planes in LDS, as the decode GEMV's prologue does for its one x;
// then a lane owns one 64-weight unit of MD_R rows per step (lpr = K / 64
// lanes per row) and dots them with each pair's planes in turn (x read from
// LDS once per step and pair, for MD_R rows).  The
// next step's weights are in flight while the current one is computed.
// Results: the f32 dot product up to the order of the sums and x to 2^-22 of
// its group maximum (the decode GEMV's bound).
constexpr int MD_R = 4;
template <int LPR>
__global__ __launch_bounds__(WG) void mt_dot4_kernel(MtGemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) u32x4 md_smem[];
    constexpr int NP = MT_MFMA_FEW, NWV = WG / WAVE, GPW = WAVE / LPR;  // lane groups per wave
    const bool second = a.mat_items > 0 && (int)blockIdx.x >= a.mat_items;
    const int it = second ? (int)blockIdx.x - a.mat_items : (int)blockIdx.x;
    if (it >= *a.nitems) return;
    const int K = a.K, U = K >> 6;  // U == LPR: one unit per lane
    const int e = a.items[2 * it], slice = a.items[2 * it + 1] >> 16;
    const int base = a.off[e] + slice * NP, n = min(NP, a.cnt[e] - slice * NP);
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE, grp = lane / LPR, j = lane % LPR;
    const DMat m = sub_rows(second ? a.m2 : a.m, e * a.rows, a.rows);
    float *y = second ? a.y2 : a.y;
    // per pair: planes [3][K/16] chunks, then xs, s32 [K/32], s16 [K/16]
    const int pstride = 3 * (K / 16) + (K / 32 * 2 + K / 16) / 4;  // in u32x4
    auto xq = [&](int pj) {
        u32x4 *b = md_smem + pj * pstride;
        float *f = (float *)(b + 3 * (K / 16));
        return XQ{b, b + K / 16, b + 2 * (K / 16), f, f + K / 32, f + K / 16};
    };
    // the first step's weights, then x (the loads are independent)
    const int rows_step = GPW * MD_R, nstep = a.rows / (rows_step * NWV);  // rows % (rows_step * NWV) == 0
    constexpr int NSTG = 2;  // ring stages: the next step in flight while one is computed
    WQ4K ring[NSTG][MD_R];
    auto issue = [&](int st, WQ4K (&w)[MD_R]) {
        const int s2 = min(st, nstep - 1), r0 = (s2 * NWV + wave) * rows_step + grp * MD_R;
#pragma unroll
        for (int r = 0; r < MD_R; r++) wload(m, r0 + r, j, w[r]);
    };
#pragma unroll
    for (int i = 0; i < NSTG - 1; i++) issue(i, ring[i]);
    // every pair's x (and x2) requested before any is used: K / 4 float4 per
    // pair, XI per thread (a loop of load-then-use would wait for each pair)
    constexpr int XI = LPR * 64 / 4 / WG > 0 ? LPR * 64 / 4 / WG : 1;
    float4 xv[NP][XI], uv[NP][XI];
#pragma unroll
    for (int pj = 0; pj < NP; pj++) {
        const size_t xo = (size_t)(a.list[base + min(pj, n - 1)] / a.xdiv) * K;
#pragma unroll
        for (int i = 0; i < XI; i++) {
            const int c = min(tid + i * WG, K / 4 - 1);
            xv[pj][i] = ((const float4 *)(a.x + xo))[c];
            uv[pj][i] = a.x2 ? ((const float4 *)(a.x2 + xo))[c] : float4{0.f, 0.f, 0.f, 0.f};
        }
    }
#pragma unroll
    for (int pj = 0; pj < NP; pj++) {
        if (pj >= n) break;
        const XQ q = xq(pj);
#pragma unroll
        for (int i = 0; i < XI; i++) {
            const int c = tid + i * WG;  // K / 4 float4, groups of 8 threads
            if (c >= K / 4) break;
            float4 v = xv[pj][i];
            if (a.x2) {  // SwiGLU (infer/forward.odin:128-132)
#pragma clang fp contract(off)
                const float4 u = uv[pj][i];
                v.x *= 1.0f / (1.0f + expf(-v.x));
                v.y *= 1.0f / (1.0f + expf(-v.y));
                v.z *= 1.0f / (1.0f + expf(-v.z));
                v.w *= 1.0f / (1.0f + expf(-v.w));
                v.x *= u.x;
                v.y *= u.y;
                v.z *= u.z;
                v.w *= u.w;
            }
            quant4(v, c, (uint32_t *)q.hi, (uint32_t *)q.mid, (uint32_t *)q.lo, (float *)q.xs, (float *)q.s32,
                   (float *)q.s16);
        }
    }
    // results [pair][row] in LDS, written out coalesced at the end (stores in
    // the loop would share the memory counter with the weight loads)
    float *yl = (float *)(md_smem + NP * pstride);
    __syncthreads();
    auto compute = [&](int st, const WQ4K (&w)[MD_R]) {
        const int r0 = (st * NWV + wave) * rows_step + grp * MD_R;
#pragma unroll 1
        for (int pj = 0; pj < n; pj++) {  // one pair's x slice live at a time
            XU4K xu;
            xload(xq(pj), j, xu);
            float acc[MD_R];
#pragma unroll
            for (int r = 0; r < MD_R; r++) acc[r] = lane_group_sum(wdot(w[r], j, xu), LPR);
            if (j == 0) {
#pragma unroll
                for (int r = 0; r < MD_R; r++) yl[pj * a.rows + r0 + r] = acc[r];
            }
        }
    };
    // NSTG steps per pass, so each stage index is static; every pass issues
    // the same loads (clamped to the last step), only the computation stops
    for (int st = 0; st < nstep; st += NSTG) {
#pragma unroll
        for (int i = 0; i < NSTG; i++) {
            issue(st + i + NSTG - 1, ring[(i + NSTG - 1) % NSTG]);
            if (st + i < nstep) compute(st + i, ring[i]);
        }
    }
    __syncthreads();
    for (int pj = 0; pj < n; pj++) {
        float *yr = y + (size_t)a.list[base + pj] * a.rows;
        for (int r = tid; r < a.rows; r += WG) yr[r] = yl[pj * a.rows + r];
    }
}

bool mt_dot4_supported(const DMat &m, int32_t K, int32_t rows) {
    const int U = K / 64;
    return m.type == T_Q4_K && m.cols == K && K % 256 == 0 && (U == 8 || U == 16 || U == 32 || U == 64) &&
           rows % ((WAVE / U) * MD_R * (WG / WAVE)) == 0 && K <= 4096;
}

hipError_t launch_mt_dot4(const MtGemvArgs &a, int max_items, hipStream_t st) {
    if (!mt_dot4_supported(a.m, a.K, a.rows) || (a.swiglu && (!mt_dot4_supported(a.m2, a.K, a.rows) || !a.y2)) ||
        a.pair_slice != MT_MFMA_FEW || a.tiles != 1 || a.xdiv <= 0 || max_items <= 0 || a.dense_n > 0)
        return hipErrorInvalidValue;
    MtGemvArgs b = a;
    b.mat_items = a.swiglu ? max_items : 0;  // gate into y, up into y2 (the SwiGLU is the consumer's)
    const int K = a.K;
    const size_t lds = (size_t)MT_MFMA_FEW * (3 * (K / 16) * 16 + (K / 32) * 8 + (K / 16) * 4) +
                       (size_t)MT_MFMA_FEW * a.rows * 4;  // x planes, then the results
    if (lds > 96 * 1024) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(a.swiglu ? 2 * max_items : max_items));
    switch (K / 64) {
    case 8: hipLaunchKernelGGL(mt_dot4_kernel<8>, grid, dim3(WG), lds, st, b); break;
    case 16: hipLaunchKernelGGL(mt_dot4_kernel<16>, grid, dim3(WG), lds, st, b); break;
    case 32: hipLaunchKernelGGL(mt_dot4_kernel<32>, grid, dim3(WG), lds, st, b); break;
    default: hipLaunchKernelGGL(mt_dot4_kernel<64>, grid, dim3(WG), lds, st, b); break;
    }
    return hipGetLastError();
}

// mt_q4i8_kernel: the same few-pair items on the matrix cores
// (v_mfma_i32_16x16x32_i8).  Each pair's x row (silu(x) * x2 when x2 is set)
// is scaled by one factor per row, s = max|x| / QI_MAX, to integers below
// 2^28 (rounded from the f32 product, so within 2^-24 of the row maximum)
// and split into four 7-bit planes, the top one signed: x = s (2^21 h +
// 2^14 p2 + 2^7 p1 + p0).  The 16 rows of the MFMA's A operand are (plane,
// pair); its B operand is 16 weight rows' 4-bit quants of one 32-weight group
// as they are stored (the low nibbles of a 64-weight unit are its first
// group, the high nibbles its second), so the weights need two logic
// operations per 8 bytes.  Per group the integer products are scaled by the
// row's 6-bit group scale in int32 (|sum| < 2^31 over a super-block), per
// super-block by d in f32; the min term, dmin m_g sum(x over the group), runs
// beside it in f32.  An item is (expert, pair slice, row tile of rows /
// tiles rows, one matrix); each of its 8 waves takes 16-row tiles of it
// (lane (n, G): row n; plane G of the four pairs for the products, pair G for
// the min term) and walks K SBS super-blocks per step with the next step's
// weights in flight.  The quants pass through a per-wave LDS staging area, so
// the loads follow the memory rather than the operand: with SBS = 2 a row's
// two super-blocks are one 128-byte line per quant plane, and each load
// instruction reads 8 such lines whole (8 lanes per line; 2 x 64 bytes per
// line at SBS = 1, which left half of each line to a second request and held
// the loads alone to ~4 TB/s), while the operand takes 8 bytes of each of four
// units.  The super-block headers of a tile (16 rows x NSB x 16 contiguous
// bytes) are loaded whole, one tile ahead, NSB dwords per lane (HT = NSB, when
// a tile takes more than one step and NSB divides 4 SBS, so that each step's
// headers sit in fixed registers of known lanes: NSB = 4, 8), and each step
// takes its rows' headers from those lanes by ds_bpermute; loaded per step
// instead (16 rows x 32 bytes, a quarter of 16 lines) they cost a fifth of the
// stream's time for a ninth of its bytes.  Otherwise (HT = 0) the headers pass
// through the staging rows.  The planes are combined across lanes at the end
// of a tile into one result per lane (row n, pair G), held in registers until
// the last tile (stores in the loop would share the memory counter with the
// weight loads).
constexpr int QI_MAXT = 16;            // 16-row tiles per wave (rows of an item <= 16 * 16 * waves)
typedef int i32x4 __attribute__((ext_vector_type(4)));
// staging row stride in bytes: SBS x 4 units of 32 quant bytes (plane 0, then
// plane 1), SBS x 16 header bytes (when HT = 0), 16 bytes against bank conflicts
__host__ __device__ constexpr int qi_srow(int sbs, int ht) { return sbs * (ht ? 128 : 144) + 16; }
// XQ: the x rows were quantized once per row (qi_quant_row, in the residual
// add + norm that wrote them: the same planes, group sums and scale this
// prologue would compute), so the prologue
// only copies each pair's 16-byte operand slots, sums and scale into LDS (one
// barrier, no arithmetic) -- every item of a chunk otherwise requantized the
// same token rows.
template <int XI, int NWV, int SBS, int HT, bool XQ = false>
__global__ __launch_bounds__(NWV * WAVE) void mt_q4i8_kernel(MtGemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) u32x4 md_smem[];
    constexpr int NP = MT_MFMA_FEW, QW = NWV * WAVE, NSTG = 2, SROW = qi_srow(SBS, HT), RPI = 16 / SBS;
    static_assert(NP == 4, "the A operand's 16 rows are 4 planes x 4 pairs");
    static_assert(SBS == 1 || SBS == 2, "one or two super-blocks per step");
    static_assert(HT == 0 || ((4 * SBS) % HT == 0 && HT % 2 == 0), "a step's headers in fixed registers");
    const bool second = a.mat_items > 0 && (int)blockIdx.x >= a.mat_items;
    const int it = second ? (int)blockIdx.x - a.mat_items : (int)blockIdx.x;
    if (it >= *a.nitems) return;
    const int K = a.K, U = K >> 6, NSB = K >> 8, NSS = NSB / SBS;  // NSB % SBS == 0
    const int e = a.items[2 * it], slice = a.items[2 * it + 1] >> 16, tile = a.items[2 * it + 1] & 0xFFFF;
    const int base = a.off[e] + slice * NP, n = min(NP, a.cnt[e] - slice * NP);
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE, G = lane >> 4;
    const int rows = a.rows / a.tiles, row0 = tile * rows;
    const DMat m = sub_rows(second ? a.m2 : a.m, e * a.rows + row0, rows);
    float *y = (second ? a.y2 : a.y) + row0;
    // LDS: the A operand [unit][lane] (16 B per lane: group g = lane / 16 of
    // the unit's first 32 weights, then of its second), the group sums
    // [pair][K/32], the scales and the wave maxima, the waves' staging rows
    u32x4 *xa = md_smem;
    float *xsum = (float *)(xa + U * WAVE);
    float *xsc = xsum + NP * (K / 32);  // [NP] scales, then [NWV][NP] wave maxima
    uint8_t *stg = (uint8_t *)(xsc + NP + NWV * NP) + wave * 16 * SROW;  // the wave's weight staging
    struct Step {
        u32x4 q[2 * SBS];  // [plane][instruction]
        uint32_t h[HT > 0 ? 1 : SBS];
    };
    const int nstep = (rows / (16 * NWV)) * NSS;  // rows % (16 NWV) == 0
    // load lanes: row ln of each instruction's RPI rows, 16-byte unit lc of the
    // row's SBS super-blocks; header lanes: row lane / 4, SBS dwords (lane % 4)
    // of its SBS x 16 header bytes
    const int ln = lane % RPI, lc = lane / RPI;
    auto issue = [&](int s, Step &w) {
        const int s2 = min(s, nstep - 1), ti = s2 / NSS, ss = s2 - ti * NSS;
        const int rb = (ti * NWV + wave) * 16;
#pragma unroll
        for (int i = 0; i < SBS; i++) {
            const size_t ui = (size_t)(rb + i * RPI + ln) * U + 4 * SBS * ss + lc;
            w.q[i] = *(const u32x4 *)(m.q + ui * 16);
            w.q[SBS + i] = *(const u32x4 *)(m.q + m.plane + ui * 16);
        }
        if constexpr (HT == 0) {
            const uint32_t *hp =
                (const uint32_t *)(m.s + ((size_t)(rb + (lane >> 2)) * NSB + SBS * ss) * 16) + (lane & 3) * SBS;
            if constexpr (SBS == 2) {
                const u32x2 hv = *(const u32x2 *)hp;
                w.h[0] = hv.x;
                w.h[1] = hv.y;
            } else {
                w.h[0] = *hp;
            }
        }
    };
    // the tile headers (HT > 0): lane l holds row l / 4's dwords [(l % 4) HT, (l % 4 + 1) HT)
    const int ntl = rows / (16 * NWV);
    uint32_t hreg[HT > 0 ? HT : 1];
    auto hload = [&](int ti) {
        if constexpr (HT > 0) {
            const uint32_t *hp =
                (const uint32_t *)(m.s + (size_t)((min(ti, ntl - 1) * NWV + wave) * 16) * HT * 16) + lane * HT;
#pragma unroll
            for (int j = 0; j < HT; j += 4) {
                if (HT - j >= 4) {
                    const u32x4 v = *(const u32x4 *)(hp + j);
                    hreg[j] = v.x; hreg[j + 1] = v.y; hreg[j + 2] = v.z; hreg[j + 3] = v.w;
                } else {
                    const u32x2 v = *(const u32x2 *)(hp + j);
                    hreg[j] = v.x; hreg[j + 1] = v.y;
                }
            }
        }
    };
    // a step's headers (HT > 0): dword c of super-block sb of row n is held by
    // lane 4 n + (4 sb + c) / HT, in hreg[(4 sb + c) % HT]
    auto gather = [&](int s, u32x4 (&hv)[SBS]) {
        if constexpr (HT > 0) {
            const int ss = s % NSS, src = 4 * (lane & 15) + (4 * SBS * ss) / HT;
#pragma unroll
            for (int hb = 0; hb < SBS; hb++) {
                uint32_t d4[4];
#pragma unroll
                for (int c = 0; c < 4; c++)
                    d4[c] = (uint32_t)__builtin_amdgcn_ds_bpermute((src + (4 * hb + c) / HT) << 2,
                                                                   (int)hreg[(4 * hb + c) % HT]);
                hv[hb] = u32x4{d4[0], d4[1], d4[2], d4[3]};
            }
        }
    };
    Step ring[NSTG];
    // every pair's x (and x2) requested before any is used, and before the
    // first weights (the loads return in order: behind the weights, the x
    // rows of 8 waves took ~7 us to arrive, ~4 us ahead of them)
    float4 xv[XQ ? 1 : NP][XI], uv[XQ ? 1 : NP][XI];
    u32x4 qv[XQ ? 4 * XI : 1];  // XQ: this thread's operand slots (U * WAVE = 4 XI QW)
    float qsum = 0.f, qscale = 0.f;
    if constexpr (XQ) {
        // the pairs' rows (uniform loads; absent pairs repeat the last), then
        // slot idx = (unit u, lane l): plane (l >> 2) & 3 of pair l & 3, lane group l >> 4
        int prow[NP];
#pragma unroll
        for (int pj = 0; pj < NP; pj++) prow[pj] = a.list[base + min(pj, n - 1)] / a.xdiv;
        const int lp = lane & 3, myrow = lp == 0 ? prow[0] : lp == 1 ? prow[1] : lp == 2 ? prow[2] : prow[3];
#pragma unroll
        for (int k = 0; k < 4 * XI; k++) {
            const int idx = tid + k * QW, u = idx / WAVE;
            qv[k] = ((const u32x4 *)a.xq)[((size_t)myrow * U + min(u, U - 1)) * 16 + (lane >> 4) * 4 + ((lane >> 2) & 3)];
        }
        const int G32 = K / 32, pj = min(tid / G32, NP - 1);  // NP * G32 <= QW for K <= 4096
        const int srow = pj == 0 ? prow[0] : pj == 1 ? prow[1] : pj == 2 ? prow[2] : prow[3];
        qsum = a.xq_sum[(size_t)srow * G32 + tid % G32];
        qscale = a.xq_scale[lp == 0 ? prow[0] : lp == 1 ? prow[1] : lp == 2 ? prow[2] : prow[3]];
    } else {
#pragma unroll
        for (int pj = 0; pj < NP; pj++) {
            const size_t xo = (size_t)(a.list[base + min(pj, n - 1)] / a.xdiv) * K;
#pragma unroll
            for (int i = 0; i < XI; i++) {
                const int c = min(tid + i * QW, K / 4 - 1);
                xv[pj][i] = ((const float4 *)(a.x + xo))[c];
                uv[pj][i] = a.x2 ? ((const float4 *)(a.x2 + xo))[c] : float4{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
    hload(0);
#pragma unroll
    for (int i = 0; i < NSTG - 1; i++) issue(i, ring[i]);
    if constexpr (XQ) {
        // (operand rows of absent pairs hold the last pair's values; their results are not stored)
#pragma unroll
        for (int k = 0; k < 4 * XI; k++)
            if (tid + k * QW < U * WAVE) xa[tid + k * QW] = qv[k];
        if (tid < NP * (K / 32)) xsum[tid] = qsum;
        if (tid < NP) xsc[tid] = qscale;
        __syncthreads();
    } else {
        float amax[NP];
#pragma unroll
        for (int pj = 0; pj < NP; pj++) {
            amax[pj] = 0.f;
#pragma unroll
            for (int i = 0; i < XI; i++) {
                float4 v = xv[pj][i];
                if (a.x2) {  // SwiGLU (infer/forward.odin:128-132)
#pragma clang fp contract(off)
                    const float4 u = uv[pj][i];
                    v.x *= 1.0f / (1.0f + expf(-v.x));
                    v.y *= 1.0f / (1.0f + expf(-v.y));
                    v.z *= 1.0f / (1.0f + expf(-v.z));
                    v.w *= 1.0f / (1.0f + expf(-v.w));
                    v.x *= u.x;
                    v.y *= u.y;
                    v.z *= u.z;
                    v.w *= u.w;
                    xv[pj][i] = v;
                }
                if (tid + i * QW < K / 4)
                    amax[pj] = fmaxf(amax[pj], fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
            amax[pj] = wave_max_all(amax[pj]);
            if (lane == 0) xsc[NP + wave * NP + pj] = amax[pj];
        }
        __syncthreads();
#pragma unroll
        for (int pj = 0; pj < NP; pj++) {
            float mx = 0.f;
#pragma unroll
            for (int w = 0; w < NWV; w++) mx = fmaxf(mx, xsc[NP + w * NP + pj]);
            const float inv = mx > 0.f ? QI_MAX / mx : 0.f;
#pragma unroll
            for (int i = 0; i < XI; i++) {
                const int c = tid + i * QW;  // float4 c: elements 4c..4c+3 (K / 4 is a multiple of 64: whole waves)
                if (c >= K / 4) break;
                const float4 v = xv[pj][i];
                const float sum = (v.x + v.y) + (v.z + v.w);
                const float sum16 = dpp_sum4(sum);
                const float sum32 = sum16 + dpp_mirror8(sum16);  // the 8 lanes of one 32-element group
                if ((c & 7) == 0) xsum[pj * (K / 32) + (c >> 3)] = sum32;
                const int q[4] = {(int)rintf(v.x * inv), (int)rintf(v.y * inv), (int)rintf(v.z * inv),
                                  (int)rintf(v.w * inv)};
                // unit c / 16, group g = (c / 2) % 4 of its first (c % 16 < 8) or second half
                uint32_t *cell = (uint32_t *)(xa + (c >> 4) * WAVE + ((c >> 1) & 3) * 16) + ((c >> 3) & 1) * 2 + (c & 1);
#pragma unroll
                for (int pl = 0; pl < 4; pl++) {
                    const int sh = 21 - 7 * pl;
                    uint32_t b = 0;
#pragma unroll
                    for (int k = 0; k < 4; k++) b |= ((uint32_t)(q[k] >> sh) & (pl == 0 ? 0xFFu : 0x7Fu)) << (8 * k);
                    cell[(4 * pl + pj) * 4] = b;  // A row 4 plane + pair
                }
            }
            if (tid == 0) xsc[pj] = mx / QI_MAX;
        }
        __syncthreads();
    }
    float facc[4] = {0.f, 0.f, 0.f, 0.f}, fmin = 0.f;
    float res[QI_MAXT];  // tile results, the latest last
#pragma unroll
    for (int k = 0; k < QI_MAXT; k++) res[k] = 0.f;
    const float pw = G == 0 ? 2097152.f : G == 1 ? 16384.f : G == 2 ? 128.f : 1.f;  // plane weight 2^(21 - 7 G)
    auto compute = [&](int s, const Step &w, const u32x4 (&hg)[SBS]) {
        const int ti = s / NSS, ss = s - ti * NSS;
        // through the wave's LDS rows (one wave's LDS operations complete in
        // order): lane (n, g) then takes dwords 2g, 2g+1 of each unit, the B
        // operand layout (group g = the unit's weights 8g .. 8g+7 of each half)
        asm volatile("" ::: "memory");  // the previous step's reads stay before these writes
#pragma unroll
        for (int i = 0; i < SBS; i++) {
            uint8_t *wr = stg + (i * RPI + ln) * SROW + lc * 32;
            *(u32x4 *)wr = w.q[i];
            *(u32x4 *)(wr + 16) = w.q[SBS + i];
        }
        if constexpr (HT == 0) {
            uint8_t *wh = stg + (lane >> 2) * SROW + SBS * 128 + (lane & 3) * SBS * 4;
            if constexpr (SBS == 2) *(u32x2 *)wh = u32x2{w.h[0], w.h[1]};
            else *(uint32_t *)wh = w.h[0];
        }
        const uint8_t *sr = stg + (lane & 15) * SROW;
#pragma unroll
        for (int hb = 0; hb < SBS; hb++) {
            const int sb = SBS * ss + hb;
            const u32x4 hv = HT > 0 ? hg[hb] : *(const u32x4 *)(sr + SBS * 128 + hb * 16);
            u32x2 wq[4];
#pragma unroll
            for (int k = 0; k < 4; k++) wq[k] = *(const u32x2 *)(sr + (4 * hb + k) * 32 + 8 * G);
            const float d = h2f(hv.x & 0xFFFFu), dmin = h2f(hv.x >> 16);
            i32x4 iacc = {0, 0, 0, 0};
            float mf = 0.f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int u = 4 * sb + k;
                uint32_t sc0, m0, sc1, m1;
                q4k_scales(k, hv.y, hv.z, hv.w, sc0, m0, sc1, m1);
                const u32x4 xo = xa[u * WAVE + lane];
                const uint32_t lo0 = wq[k].x & 0x0F0F0F0Fu, lo1 = wq[k].y & 0x0F0F0F0Fu;
                const uint32_t hi0 = (wq[k].x >> 4) & 0x0F0F0F0Fu, hi1 = (wq[k].y >> 4) & 0x0F0F0F0Fu;
                const i32x4 z = {0, 0, 0, 0};
                const i32x4 dA = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                    (long)(((uint64_t)xo.y << 32) | xo.x), (long)(((uint64_t)lo1 << 32) | lo0), z, 0, 0, 0);
                const i32x4 dB = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                    (long)(((uint64_t)xo.w << 32) | xo.z), (long)(((uint64_t)hi1 << 32) | hi0), z, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++) iacc[v] += __mul24((int)sc0, dA[v]) + __mul24((int)sc1, dB[v]);  // |dA| < 2^23
                const float2 xs2 = *(const float2 *)&xsum[G * (K / 32) + 2 * u];
                mf += (float)m0 * xs2.x + (float)m1 * xs2.y;
            }
#pragma unroll
            for (int v = 0; v < 4; v++) facc[v] += d * (float)iacc[v];
            fmin += dmin * mf;
        }
        if (ss == NSS - 1) {  // the tile's row n = lane % 16 is done: combine the planes
            float t[4];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                t[v] = pw * facc[v];
                t[v] += __shfl_xor(t[v], 16, WAVE);
                t[v] += __shfl_xor(t[v], 32, WAVE);
                facc[v] = 0.f;
            }
            const float S = G == 0 ? t[0] : G == 1 ? t[1] : G == 2 ? t[2] : t[3];
#pragma unroll
            for (int k = 0; k + 1 < QI_MAXT; k++) res[k] = res[k + 1];
            res[QI_MAXT - 1] = xsc[G] * S - fmin;
            fmin = 0.f;
        }
    };
    // NSTG steps per pass, so each stage index is static; every pass issues
    // the same loads (clamped to the last step), only the computation stops
    // (HT > 0: a step's headers are taken before the next tile's are requested
    // into the same registers, at the tile's last step)
    for (int st = 0; st < nstep; st += NSTG) {
#pragma unroll
        for (int i = 0; i < NSTG; i++) {
            const int s = st + i;
            u32x4 hg[SBS];
            if (HT > 0 && s < nstep) {
                gather(s, hg);
                if (s % NSS == NSS - 1) hload(s / NSS + 1);
            }
            issue(s + NSTG - 1, ring[(i + NSTG - 1) % NSTG]);
            if (s < nstep) compute(s, ring[i], hg);
        }
    }
    if (G < n) {  // the wave's tiles: tile i's result is res[QI_MAXT - ntl + i]
        float *yr = y + (size_t)a.list[base + G] * a.rows + wave * 16 + (lane & 15);
#pragma unroll
        for (int k = 0; k < QI_MAXT; k++) {
            const int i = k - (QI_MAXT - ntl);
            if (i >= 0) yr[(size_t)i * NWV * 16] = res[k];
        }
    }
}

constexpr int QI_NW = 8;  // waves per workgroup: the x planes in LDS serve 8 waves (4 measured 2% slower)
static int qi_sbs(int32_t K) { return (K / 256) % 2 == 0 ? 2 : 1; }
// headers per tile when a tile takes more than one step and NSB divides 4 SBS
// (NSB = 4, 8 here), else per step (at NSB = 2 a step's headers are already
// 512 contiguous bytes, and the permutes only cost)
static int qi_ht(int32_t K) {
    const int nsb = K / 256;
    return qi_sbs(K) == 2 && (nsb == 4 || nsb == 8) ? nsb : 0;
}
static size_t mt_q4i8_lds(int32_t K, int nw) {
    return (size_t)(K / 64) * WAVE * 16 + (size_t)MT_MFMA_FEW * (K / 32) * 4 +
           (size_t)(MT_MFMA_FEW + nw * MT_MFMA_FEW) * 4 + (size_t)nw * 16 * qi_srow(qi_sbs(K), qi_ht(K));
}

// rows: the rows of one row tile
bool mt_q4i8_supported(const DMat &m, int32_t K, int32_t rows) {
    return m.type == T_Q4_K && m.cols == K && K % 256 == 0 && K <= 4096 && rows > 0 && rows % (16 * QI_NW) == 0 &&
           rows <= QI_MAXT * 16 * QI_NW;
}

hipError_t launch_mt_q4i8(const MtGemvArgs &a, int max_items, hipStream_t st) {
    if (a.tiles < 1 || a.rows % a.tiles || !mt_q4i8_supported(a.m, a.K, a.rows / a.tiles) ||
        (a.swiglu && (!mt_q4i8_supported(a.m2, a.K, a.rows / a.tiles) || !a.y2)) || a.m.rows < a.rows ||
        a.pair_slice != MT_MFMA_FEW || a.xdiv <= 0 || max_items <= 0 || a.dense_n > 0)
        return hipErrorInvalidValue;
    MtGemvArgs b = a;
    b.mat_items = a.swiglu ? max_items : 0;  // gate into y, up into y2 (the SwiGLU is the consumer's)
    const size_t lds = mt_q4i8_lds(a.K, QI_NW);
    const dim3 grid((unsigned)(a.swiglu ? 2 * max_items : max_items)), block(QI_NW * WAVE);
    const bool x1 = a.K <= 4 * QI_NW * WAVE;  // K <= 2048: NSB <= 8
    if (a.xq && !a.x2) {
        if (!a.xq_sum || !a.xq_scale) return hipErrorInvalidValue;
        switch (x1 ? qi_ht(a.K) : -1) {
        case 8: hipLaunchKernelGGL((mt_q4i8_kernel<1, QI_NW, 2, 8, true>), grid, block, lds, st, b); break;
        case 4: hipLaunchKernelGGL((mt_q4i8_kernel<1, QI_NW, 2, 4, true>), grid, block, lds, st, b); break;
        case 0:
            if (qi_sbs(a.K) == 2) hipLaunchKernelGGL((mt_q4i8_kernel<1, QI_NW, 2, 0, true>), grid, block, lds, st, b);
            else hipLaunchKernelGGL((mt_q4i8_kernel<1, QI_NW, 1, 0, true>), grid, block, lds, st, b);
            break;
        default:
            if (qi_sbs(a.K) == 2) hipLaunchKernelGGL((mt_q4i8_kernel<2, QI_NW, 2, 0, true>), grid, block, lds, st, b);
            else hipLaunchKernelGGL((mt_q4i8_kernel<2, QI_NW, 1, 0, true>), grid, block, lds, st, b);
            break;
        }
        return hipGetLastError();
    }
    switch (x1 ? qi_ht(a.K) : -1) {
    case 8: hipLaunchKernelGGL((mt_q4i8_kernel<1, QI_NW, 2, 8>), grid, block, lds, st, b); break;
    case 4: hipLaunchKernelGGL((mt_q4i8_kernel<1, QI_NW, 2, 4>), grid, block, lds, st, b); break;
    case 0:
        if (qi_sbs(a.K) == 2) hipLaunchKernelGGL((mt_q4i8_kernel<1, QI_NW, 2, 0>), grid, block, lds, st, b);
        else hipLaunchKernelGGL((mt_q4i8_kernel<1, QI_NW, 1, 0>), grid, block, lds, st, b);
        break;
    default:
        if (qi_sbs(a.K) == 2) hipLaunchKernelGGL((mt_q4i8_kernel<2, QI_NW, 2, 0>), grid, block, lds, st, b);
        else hipLaunchKernelGGL((mt_q4i8_kernel<2, QI_NW, 1, 0>), grid, block, lds, st, b);
        break;
    }
    return hipGetLastError();
}

}  // namespace oi
