// gemm.hip -- batched projection for prefill on gfx950 matrix cores:
//   C[t][r] = sum_k f16(dequant(W)[r][k]) * X[t][k]     (f32 accumulate)
// for n tokens t at once (reference: the batched-prefill MMQ kernels
// qwen3_5/metal.odin:493-609 and gemm_harness/gemm_test.odin:97-135, 297-337,
// which stage both operands in half precision and accumulate in float).
// X is token-major f16 [n][K], C token-major f32 [n][M] (the transposes of the
// reference harness's B[K][N] and C[M][N]; same products).
//
// Work layout: a workgroup of 8 waves (two per SIMD, so that one wave's
// dequantization overlaps the other's matrix and LDS work) computes 128 rows x
// 64 tokens over a slice of K; wave w holds rows 16w .. 16w+15 in four
// v_mfma_f32_16x16x32_f16 accumulators (16 tokens each).  K is walked in
// chunks of 256 (one Q4_K / Q6_K super-block, eight Q8_0 blocks); the chunk's
// 64 x 256 activations are staged in LDS once per workgroup and read by all
// four waves.  Every lane dequantizes the weights it feeds to the matrix cores
// straight from the plane layout (no LDS staging of W): lane quarter q owns one
// 64-weight unit of the chunk (16-byte plane loads), and the chunk's eight
// 32-wide K steps take 8 of its weights each.  The K order inside a chunk is a
// permutation chosen so that each lane's bytes are contiguous; the activation
// octets are placed by the same permutation (omap), so every product pairs
// the right weight with the right activation.
// Dequantization follows ggml/quant.odin exactly (separately rounded products,
// (d*sc)*q for Q6_K), then rounds to f16 (RNE), as the reference's staging.
//
// The FFN's gate and up projections can run as one pass (gemm_q_kernel<G, 2>,
// launch_gemm_swiglu) that writes the f16 SwiGLU of the pair instead of two
// f32 products.
//
// Operand layout of v_mfma_f32_16x16x32_f16 (per lane l, 8 halves each):
//   A[i][k]: i = l % 16, k = 8 (l / 16) + e;  B[k][j]: j = l % 16, k = 8 (l / 16) + e
//   D[i][j] (4 floats): j = l % 16, i = 4 (l / 16) + e.

#include <algorithm>

#include "device_common.h"

namespace oi {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

typedef __amdgpu_buffer_rsrc_t rsrc_t;
// raw buffer descriptors (data format 32, the gfx9 value for untyped access):
// 32-bit per-lane offsets and a uniform per-chunk offset, so the loads need no
// 64-bit address arithmetic; reads past `bytes` return zero
static __device__ __forceinline__ rsrc_t make_rsrc(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)(uint32_t)bytes, 0x00020000);
}
static __device__ __forceinline__ u32x4 bld16(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

constexpr int GM_WAVES = 8, GM_RT = 1, GM_ROWS = 16 * GM_RT * GM_WAVES, GM_TOK = 64, GM_THREADS = GM_WAVES * WAVE;
constexpr int GM_KC = 256;                  // K per chunk
constexpr int GM_XV = GM_TOK * GM_KC / 8;   // 16-byte activation pieces per chunk
constexpr int GM_XPT = GM_XV / GM_THREADS;  // ... per thread
constexpr int GM_WD = 2;                    // weight chunks in the register ring (1 in flight)

// one projection of a multi-projection launch: its matrix, partial products
// ([split][n][rows]), K chunks per slice, row tiles, and its first block
struct GemmSeg {
    DMat m;
    float *c;
    int32_t cps, nx, first;
};
constexpr int GM_MAX_SEG = 4;
struct GemmArgs {
    DMat m;             // weights [M][K], device plane layout
    const uint16_t *x;  // [n][K] f16
    float *c;           // [n][M], or [split][n][M] partial products when K is split
    int32_t n;
    DMat m2;            // NP == 2: the up matrix (m is gate), same type and shape
    uint16_t *h;        // NP == 2: [n][M] f16 silu(gate x) * (up x)
    // nseg > 0: projections of the same x (same type and K) in one launch; a
    // flat grid whose block b belongs to the last segment with first <= b
    // (m, c and cps above are then unused)
    int32_t nseg;
    GemmSeg seg[GM_MAX_SEG];
};

// f32 -> f16 (RNE) of values already rounded to f32 (f2h: the conversion is
// kept apart from the fma that produced the value)
static __device__ __forceinline__ h8 cvt8(const float (&v)[8]) {
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; e++) r[e] = __builtin_bit_cast(_Float16, f2h(v[e]));
    return r;
}
static __device__ __forceinline__ uint32_t byte_of(uint32_t lo, uint32_t hi, int e) {
    return ((e < 4 ? lo : hi) >> (8 * (e & 3))) & 0xFFu;
}
// keeps a masked word opaque, so that its bytes convert with v_cvt_f32_ubyte{0..3}
// instead of being re-extracted one by one from the unmasked word
static __device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// ---- per-type raw loads and step dequantization ------------------------------
// raw(): the bytes lane quarter q needs for chunk c of one row (issued chunks
// ahead); deq(): the 8 weights of K step st as the A operand; omap(q, st): the
// activation octet (8 consecutive K) those weights multiply.

// Lane offsets: Off holds the per-lane byte offsets of one row's streams,
// computed once; raw() adds the chunk's uniform offset.

// Q4_K, chunk = super-block c; quarter q owns unit 4c + q (bytes 0-15 in plane
// 0, 16-31 in plane 1).  Step st = 4h + 2p + b: nibble h (group 2q + h), plane
// p, bytes 8b .. 8b+7 of that plane; weight = 64q + 32h + 16p + 8b + e, so the
// octet is 8q + st.  ggml/quant.odin:178-209.
struct GQ4K {
    struct Src {
        rsrc_t q, s;
        uint32_t plane;
    };
    struct Off {
        uint32_t q, s;
    };
    struct Raw {
        u32x4 p0, p1, hdr;
    };
    static __device__ __forceinline__ Src src(const DMat &m) {
        return Src{make_rsrc(m.q, 2 * m.plane), make_rsrc(m.s, (size_t)m.rows * (m.cols >> 8) * 16), (uint32_t)m.plane};
    }
    static __device__ __forceinline__ Off off(const DMat &m, int row, int q) {
        return Off{(uint32_t)((row * (m.cols >> 6) + q) * 16), (uint32_t)(row * (m.cols >> 8) * 16)};
    }
    static __device__ __forceinline__ void raw(const Src &g, const Off &o, int c, Raw &r) {
        r.p0 = bld16(g.q, o.q, 64 * c);
        r.p1 = bld16(g.q, o.q + g.plane, 64 * c);
        r.hdr = bld16(g.s, o.s, 16 * c);
    }
    struct Pre {
        float d1[2], mm[2];
    };
    static __device__ __forceinline__ Pre pre(const Raw &r, int q) {
        Pre p;
        const float d = h2f(r.hdr.x & 0xFFFFu), dmin = h2f(r.hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(q, r.hdr.y, r.hdr.z, r.hdr.w, sc0, m0, sc1, m1);
        p.d1[0] = d * (float)sc0;
        p.mm[0] = dmin * (float)m0;
        p.d1[1] = d * (float)sc1;
        p.mm[1] = dmin * (float)m1;
        return p;
    }
    // d1 * nib is exact in f32 (at most 11 + 6 + 4 significant bits), so the
    // fused d1 * nib - mm rounds exactly as the separate product and difference
    static __device__ __forceinline__ h8 deq(const Raw &r, const Pre &p, int st) {
        const int h = st >> 2, pl = (st >> 1) & 1, b = st & 1;
        const u32x4 &w = pl ? r.p1 : r.p0;
        const uint32_t lo = opaque(((b ? w.z : w.x) >> (4 * h)) & 0x0F0F0F0Fu);
        const uint32_t hi = opaque(((b ? w.w : w.y) >> (4 * h)) & 0x0F0F0F0Fu);
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = __builtin_fmaf(p.d1[h], (float)byte_of(lo, hi, e), -p.mm[h]);
        return cvt8(v);
    }
    static __device__ __forceinline__ int omap(int q, int st) { return 8 * q + st; }
};

// Q6_K, chunk = super-block c; quarter q owns unit 4c + q = unit u' = q % 2 of
// half h = q / 2, bytes 0-15 of its ql-low, ql-high and qh planes.  Step
// st = 2s + b: run s (ql-low/high nibble and qh bits 2s, scale 8h + u' + 2s),
// bytes 8b .. 8b+7; weight = 128h + 32s + 16u' + 8b + e, octet
// 16h + 4s + 2u' + b.  ggml/quant.odin:212-247.
struct GQ6K {
    struct Src {
        rsrc_t q, s, d;
        uint32_t plane;
    };
    struct Off {
        uint32_t q, s, d;
    };
    struct Raw {
        u32x4 qa, qb, qh;
        u32x2 scw;
        uint32_t d;
    };
    static __device__ __forceinline__ Src src(const DMat &m) {
        const size_t nsb = (size_t)m.rows * (m.cols >> 8);
        return Src{make_rsrc(m.q, 3 * m.plane), make_rsrc(m.s, nsb * 16), make_rsrc(m.d, nsb * 2), (uint32_t)m.plane};
    }
    static __device__ __forceinline__ Off off(const DMat &m, int row, int q) {
        const int nsb = m.cols >> 8;
        return Off{(uint32_t)((row * (m.cols >> 6) + q) * 16), (uint32_t)(row * nsb * 16 + 8 * (q >> 1)),
                   (uint32_t)(row * nsb * 2)};
    }
    static __device__ __forceinline__ void raw(const Src &g, const Off &o, int c, Raw &r) {
        r.qa = bld16(g.q, o.q, 64 * c);
        r.qb = bld16(g.q, o.q + g.plane, 64 * c);
        r.qh = bld16(g.q, o.q + 2 * g.plane, 64 * c);
        r.scw = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(g.s, o.s, 16 * c, 0));
        r.d = __builtin_amdgcn_raw_buffer_load_b16(g.d, o.d, 2 * c, 0);
    }
    struct Pre {
        float ds[4], off[4];
    };
    static __device__ __forceinline__ Pre pre(const Raw &r, int q) {
        Pre p;
        const float d = h2f(r.d);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int is = (q & 1) + 2 * s;
            p.ds[s] = d * (float)(int8_t)byte_of(r.scw.x, r.scw.y, is);
            p.off[s] = -32.f * p.ds[s];
        }
        return p;
    }
    // ds * (code - 32) as one fused ds * code - 32 ds: the exact value is the
    // same and the fma rounds it once, as the reference's single product
    static __device__ __forceinline__ h8 deq(const Raw &r, const Pre &p, int st) {
        const int s = st >> 1, b = st & 1;
        const u32x4 &l = (s & 1) ? r.qb : r.qa;
        const uint32_t llo = ((b ? l.z : l.x) >> (4 * (s >> 1))) & 0x0F0F0F0Fu;
        const uint32_t lhi = ((b ? l.w : l.y) >> (4 * (s >> 1))) & 0x0F0F0F0Fu;
        const uint32_t hlo = (((b ? r.qh.z : r.qh.x) >> (2 * s)) & 0x03030303u) << 4;
        const uint32_t hhi = (((b ? r.qh.w : r.qh.y) >> (2 * s)) & 0x03030303u) << 4;
        const uint32_t wlo = opaque(llo | hlo), whi = opaque(lhi | hhi);  // 6-bit codes, one per byte
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = __builtin_fmaf(p.ds[s], (float)byte_of(wlo, whi, e), p.off[s]);
        return cvt8(v);
    }
    static __device__ __forceinline__ int omap(int q, int st) {
        return 16 * (q >> 1) + 4 * (st >> 1) + 2 * (q & 1) + (st & 1);
    }
};

// Q8_0, chunk = blocks 8c .. 8c+7; quarter q owns unit 4c + q (blocks 8c + 2q
// and 8c + 2q + 1); plane 2 blk + half holds bytes 16 half .. +15 of block blk.
// Step st = 4 blk + 2 half + b: weight 64q + 8st + e, octet 8q + st.
// ggml/quant.odin:87-96.
struct GQ80 {
    struct Src {
        rsrc_t q, d;
        uint32_t plane;
    };
    struct Off {
        uint32_t q, d;
    };
    struct Raw {
        u32x4 pl[4];
        uint32_t d;
    };
    static __device__ __forceinline__ Src src(const DMat &m) {
        return Src{make_rsrc(m.q, 4 * m.plane), make_rsrc(m.d, (size_t)m.rows * (m.cols >> 5) * 2), (uint32_t)m.plane};
    }
    static __device__ __forceinline__ Off off(const DMat &m, int row, int q) {
        return Off{(uint32_t)((row * (m.cols >> 6) + q) * 16), (uint32_t)((row * (m.cols >> 5) + 2 * q) * 2)};
    }
    static __device__ __forceinline__ void raw(const Src &g, const Off &o, int c, Raw &r) {
#pragma unroll
        for (int k = 0; k < 4; k++) r.pl[k] = bld16(g.q, o.q + k * g.plane, 64 * c);
        r.d = __builtin_amdgcn_raw_buffer_load_b32(g.d, o.d, 16 * c, 0);
    }
    struct Pre {
        float d[2];
    };
    static __device__ __forceinline__ Pre pre(const Raw &r, int) {
        return Pre{{h2f(r.d & 0xFFFFu), h2f(r.d >> 16)}};
    }
    static __device__ __forceinline__ h8 deq(const Raw &r, const Pre &p, int st) {
#pragma clang fp contract(off)
        const u32x4 &w = r.pl[st >> 1];
        const int b = st & 1;
        const uint32_t lo = b ? w.z : w.x, hi = b ? w.w : w.y;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = p.d[st >> 2] * (float)(int8_t)byte_of(lo, hi, e);
        return cvt8(v);
    }
    static __device__ __forceinline__ int omap(int q, int st) { return 8 * q + st; }
};

// One workgroup: rows [128 bx, +128), tokens [64 by, +64), chunks
// [bz * cps, +cps) of K.  Activations: chunk c + 1 is loaded into registers
// while chunk c is computed, then stored to the LDS buffer of its parity
// (piece (token j, octet o) at slot 64 o + (j ^ (o % 8)): conflict-free stores
// of 8 consecutive octets and conflict-free 16-lane operand reads); weights
// run GM_WD - 1 chunks ahead in a register ring.  With more than one K slice
// (split > 1) slice z writes its partial products to c + z n M; gemm_reduce
// sums them in slice order.
//
// NP == 2 (gate and up of the FFN, one K slice): both matrices' rows are
// computed against the same staged activations, each B operand read from LDS
// feeding both products, and the epilogue writes the f16 SwiGLU of the pair
// (infer/forward.odin:128-132: v *= 1/(1+exp(-v)); v *= up; then the half
// staging of the next projection's input).
template <class G, int NP = 1>
__global__ __launch_bounds__(GM_THREADS) void gemm_q_kernel(GemmArgs a, int cps) {
    __shared__ __attribute__((aligned(16))) u32x4 xs[2][GM_XV];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int q = lane >> 4, li = lane & 15;
    // the block's matrix, output and (row tile, token tile, K slice)
    DMat mat = a.m;
    float *cout = a.c;
    int bx = (int)blockIdx.x, by = (int)blockIdx.y, bz = (int)blockIdx.z;
    if (NP == 1 && a.nseg > 0) {
        int sg = 0;
#pragma unroll
        for (int i = 1; i < GM_MAX_SEG; i++)
            if (i < a.nseg && bx >= a.seg[i].first) sg = i;
        const GemmSeg &g = a.seg[sg];
        const int ny = (a.n + GM_TOK - 1) / GM_TOK, loc = bx - g.first;
        mat = g.m;
        cout = g.c;
        cps = g.cps;
        bz = loc / (g.nx * ny);
        by = (loc - bz * g.nx * ny) / g.nx;
        bx = loc - bz * g.nx * ny - by * g.nx;
    }
    const int M = mat.rows, K = mat.cols;
    const int rbase = bx * GM_ROWS + 16 * GM_RT * wave;
    typename G::Src src[NP];
    src[0] = G::src(mat);
    if (NP == 2) src[NP - 1] = G::src(a.m2);  // same shape: the same lane offsets
    typename G::Off off[GM_RT];
#pragma unroll
    for (int rt = 0; rt < GM_RT; rt++) off[rt] = G::off(mat, min(rbase + 16 * rt + li, M - 1), q);  // rows past M: not stored
    const int t0 = by * GM_TOK;
    const int nchunk = K / GM_KC;
    const int c0 = bz * cps, c1 = min(nchunk, c0 + cps);

    const rsrc_t xsrc = make_rsrc(a.x, (size_t)a.n * K * 2);
    uint32_t xoff[GM_XPT];
#pragma unroll
    for (int i = 0; i < GM_XPT; i++) {
        const int p = threadIdx.x + i * GM_THREADS, j = p >> 5, o = p & 31;
        xoff[i] = (uint32_t)(min(t0 + j, a.n - 1) * K * 2 + 16 * o);
    }
    u32x4 xr[GM_XPT];
    auto xfetch = [&](int c) {
#pragma unroll
        for (int i = 0; i < GM_XPT; i++) xr[i] = bld16(xsrc, xoff[i], c * GM_KC * 2);
    };
    auto xstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < GM_XPT; i++) {
            const int p = threadIdx.x + i * GM_THREADS, j = p >> 5, o = p & 31;
            xs[buf][o * GM_TOK + (j ^ (o & 7))] = xr[i];
        }
    };

    f32x4v acc[NP][GM_RT][4];
#pragma unroll
    for (int mp = 0; mp < NP; mp++)
#pragma unroll
        for (int rt = 0; rt < GM_RT; rt++)
#pragma unroll
            for (int t = 0; t < 4; t++) acc[mp][rt][t] = f32x4v{0.f, 0.f, 0.f, 0.f};
    // unconditional loads: chunks past the slice re-read its first, unused
    typename G::Raw ring[GM_WD][NP][GM_RT];
#pragma unroll
    for (int r = 0; r < GM_WD - 1; r++)
#pragma unroll
        for (int mp = 0; mp < NP; mp++)
#pragma unroll
            for (int rt = 0; rt < GM_RT; rt++)
                G::raw(src[mp], off[rt], c0 + r < c1 ? c0 + r : c0, ring[r][mp][rt]);
    if (c0 < c1) xfetch(c0);
    for (int cb = c0; cb < c1; cb += GM_WD) {
#pragma unroll
        for (int r = 0; r < GM_WD; r++) {
            const int c = cb + r;
            if (c >= c1) break;
            const int cn = c + GM_WD - 1 < c1 ? c + GM_WD - 1 : c0;
#pragma unroll
            for (int mp = 0; mp < NP; mp++)
#pragma unroll
                for (int rt = 0; rt < GM_RT; rt++) G::raw(src[mp], off[rt], cn, ring[(r + GM_WD - 1) % GM_WD][mp][rt]);
            const int buf = (c - c0) & 1;
            xstore(buf);
            if (c + 1 < c1) xfetch(c + 1);
            __syncthreads();  // chunk c staged; every wave is done with chunk c - 2's buffer
            typename G::Pre pre[NP][GM_RT];
#pragma unroll
            for (int mp = 0; mp < NP; mp++)
#pragma unroll
                for (int rt = 0; rt < GM_RT; rt++) pre[mp][rt] = G::pre(ring[r][mp][rt], q);
#pragma unroll
            for (int st = 0; st < 8; st++) {
                const int o = G::omap(q, st);
                h8 B[4];
#pragma unroll
                for (int t = 0; t < 4; t++) B[t] = __builtin_bit_cast(h8, xs[buf][o * GM_TOK + ((16 * t + li) ^ (o & 7))]);
#pragma unroll
                for (int mp = 0; mp < NP; mp++)
#pragma unroll
                    for (int rt = 0; rt < GM_RT; rt++) {
                        const h8 A = G::deq(ring[r][mp][rt], pre[mp][rt], st);
#pragma unroll
                        for (int t = 0; t < 4; t++)
                            acc[mp][rt][t] =
                                __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[t], acc[mp][rt][t], 0, 0, 0);
                    }
            }
        }
    }
    // D of tile (rt, t): lane (j, g) holds rows 4g .. 4g+3 of column (token) j
    if (NP == 2) {
#pragma unroll
        for (int rt = 0; rt < GM_RT; rt++) {
            const int r0 = rbase + 16 * rt + 4 * q;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int tk = t0 + 16 * t + li;
                if (tk >= a.n) continue;
                uint16_t hv[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
#pragma clang fp contract(off)
                    float v = acc[0][rt][t][e];
                    v *= 1.0f / (1.0f + expf(-v));
                    v *= acc[NP - 1][rt][t][e];
                    hv[e] = f2h(v);
                }
                uint16_t *dst = a.h + (size_t)tk * M + r0;
                if (r0 + 3 < M && (M & 3) == 0) {
                    *(u32x2 *)dst = u32x2{(uint32_t)hv[0] | ((uint32_t)hv[1] << 16),
                                          (uint32_t)hv[2] | ((uint32_t)hv[3] << 16)};
                    continue;
                }
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (r0 + e < M) dst[e] = hv[e];
            }
        }
        return;
    }
    float *out = cout + (size_t)bz * a.n * M;
#pragma unroll
    for (int rt = 0; rt < GM_RT; rt++) {
        const int r0 = rbase + 16 * rt + 4 * q;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int tk = t0 + 16 * t + li;
            if (tk >= a.n) continue;
            float *dst = out + (size_t)tk * M + r0;
            if (r0 + 3 < M && (M & 3) == 0) {
                *(f32x4v *)dst = acc[0][rt][t];
                continue;
            }
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (r0 + e < M) dst[e] = acc[0][rt][t][e];
        }
    }
}

// c[i] = sum over slices z (in order) of part[z][i]
__global__ __launch_bounds__(WG) void gemm_reduce(const float *part, float *c, int64_t total, int split) {
    const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (4 * i + 3 < total) {
        f32x4v s = *(const f32x4v *)(part + 4 * i);
        for (int z = 1; z < split; z++) s += *(const f32x4v *)(part + z * total + 4 * i);
        *(f32x4v *)(c + 4 * i) = s;
    } else {
        for (int64_t k = 4 * i; k < total; k++) {
            float s = part[k];
            for (int z = 1; z < split; z++) s += part[z * total + k];
            c[k] = s;
        }
    }
}

bool gemm_supported(const DMat &m) {
    return (m.type == T_Q4_K || m.type == T_Q6_K || m.type == T_Q8_0) && m.cols % GM_KC == 0;
}

static int normalize_split(int nchunk, int split) {
    const int cps = (nchunk + split - 1) / split;
    return (nchunk + cps - 1) / cps;
}

// K is split so that about 256 workgroups run (one per CU; each slice at least
// two chunks; measured best on 4096/12288 x 64 x 4096/12288), and no further
// than the partial-product buffer holds.
int gemm_split(const DMat &m, int32_t n, size_t part_bytes) {
    const int nchunk = m.cols / GM_KC;
    const int tiles = ((m.rows + GM_ROWS - 1) / GM_ROWS) * ((n + GM_TOK - 1) / GM_TOK);
    int split = std::max(1, std::min((256 + tiles / 2) / tiles, nchunk / 2));
    const size_t per = (size_t)n * m.rows * 4;
    split = (int)std::min<size_t>(split, std::max<size_t>(1, part_bytes / per));
    return normalize_split(nchunk, split);
}

// With split > 1 the slices' partial products go to `part` (split * n * rows
// floats) and gemm_reduce sums them into c.
hipError_t launch_gemm(const DMat &m, const uint16_t *x, int32_t n, float *c, float *part, size_t part_bytes,
                       hipStream_t st) {
    if (!gemm_supported(m) || n <= 0) return hipErrorInvalidValue;
    const int nchunk = m.cols / GM_KC;
    const int split = gemm_split(m, n, part ? part_bytes : 0);
    const int cps = (nchunk + split - 1) / split;
    GemmArgs a{m, x, split > 1 ? part : c, n, DMat{}, nullptr, 0, {}};
    dim3 grid((m.rows + GM_ROWS - 1) / GM_ROWS, (n + GM_TOK - 1) / GM_TOK, split), block(GM_THREADS);
    switch (m.type) {
    case T_Q4_K: hipLaunchKernelGGL(gemm_q_kernel<GQ4K>, grid, block, 0, st, a, cps); break;
    case T_Q6_K: hipLaunchKernelGGL(gemm_q_kernel<GQ6K>, grid, block, 0, st, a, cps); break;
    default: hipLaunchKernelGGL(gemm_q_kernel<GQ80>, grid, block, 0, st, a, cps); break;
    }
    if (split > 1) {
        const int64_t total = (int64_t)n * m.rows;
        const int64_t nb = ((total + 3) / 4 + WG - 1) / WG;
        hipLaunchKernelGGL(gemm_reduce, dim3((unsigned)nb), dim3(WG), 0, st, part, c, total, split);
    }
    return hipGetLastError();
}

// h[t][r] = f16(silu(gate x)[t][r] * (up x)[t][r]) in one pass over K: only
// when the projection needs no K split (gemm_split == 1 for this n)
bool gemm_swiglu_supported(const DMat &gate, const DMat &up, int32_t n) {
    return gemm_supported(gate) && up.type == gate.type && up.rows == gate.rows && up.cols == gate.cols && n > 0 &&
           gemm_split(gate, n, SIZE_MAX) == 1;
}

hipError_t launch_gemm_swiglu(const DMat &gate, const DMat &up, const uint16_t *x, int32_t n, uint16_t *h,
                              hipStream_t st) {
    if (!gemm_swiglu_supported(gate, up, n) || !h) return hipErrorInvalidValue;
    GemmArgs a{gate, x, nullptr, n, up, h, 0, {}};
    dim3 grid((gate.rows + GM_ROWS - 1) / GM_ROWS, (n + GM_TOK - 1) / GM_TOK, 1), block(GM_THREADS);
    const int cps = gate.cols / GM_KC;
    switch (gate.type) {
    case T_Q4_K: hipLaunchKernelGGL((gemm_q_kernel<GQ4K, 2>), grid, block, 0, st, a, cps); break;
    case T_Q6_K: hipLaunchKernelGGL((gemm_q_kernel<GQ6K, 2>), grid, block, 0, st, a, cps); break;
    default: hipLaunchKernelGGL((gemm_q_kernel<GQ80, 2>), grid, block, 0, st, a, cps); break;
    }
    return hipGetLastError();
}

hipError_t launch_gemm_parts(const DMat &m, const uint16_t *x, int32_t n, float *part, size_t part_bytes, int *split,
                             hipStream_t st) {
    if (!gemm_supported(m) || n <= 0 || !part || part_bytes < (size_t)n * m.rows * 4) return hipErrorInvalidValue;
    const int nchunk = m.cols / GM_KC;
    *split = gemm_split(m, n, part_bytes);
    const int cps = (nchunk + *split - 1) / *split;
    GemmArgs a{m, x, part, n, DMat{}, nullptr, 0, {}};
    dim3 grid((m.rows + GM_ROWS - 1) / GM_ROWS, (n + GM_TOK - 1) / GM_TOK, *split), block(GM_THREADS);
    switch (m.type) {
    case T_Q4_K: hipLaunchKernelGGL(gemm_q_kernel<GQ4K>, grid, block, 0, st, a, cps); break;
    case T_Q6_K: hipLaunchKernelGGL(gemm_q_kernel<GQ6K>, grid, block, 0, st, a, cps); break;
    default: hipLaunchKernelGGL(gemm_q_kernel<GQ80>, grid, block, 0, st, a, cps); break;
    }
    return hipGetLastError();
}

// launch_gemm_parts for up to GM_MAX_SEG projections of the same x in one
// launch (same type and K): the same blocks, K slices and partial products as
// one launch each, so the same results; one launch's fixed cost instead of
// nseg (the DeltaNet layer's four input projections at 64 tokens: 28.7 us in
// four launches)
hipError_t launch_gemm_parts_multi(const DMat *const *m, float *const *part, const size_t *part_bytes, int nseg,
                                   const uint16_t *x, int32_t n, int *split, hipStream_t st) {
    if (nseg < 1 || nseg > GM_MAX_SEG || n <= 0) return hipErrorInvalidValue;
    GemmArgs a{*m[0], x, nullptr, n, DMat{}, nullptr, nseg, {}};
    int blocks = 0;
    const int ny = (n + GM_TOK - 1) / GM_TOK;
    for (int i = 0; i < nseg; i++) {
        const DMat &mi = *m[i];
        if (!gemm_supported(mi) || mi.type != m[0]->type || mi.cols != m[0]->cols || !part[i] ||
            part_bytes[i] < (size_t)n * mi.rows * 4)
            return hipErrorInvalidValue;
        const int nchunk = mi.cols / GM_KC;
        split[i] = gemm_split(mi, n, part_bytes[i]);
        const int nx = (mi.rows + GM_ROWS - 1) / GM_ROWS;
        a.seg[i] = GemmSeg{mi, part[i], (nchunk + split[i] - 1) / split[i], nx, blocks};
        blocks += nx * ny * split[i];
    }
    const dim3 grid((unsigned)blocks), block(GM_THREADS);
    switch (m[0]->type) {
    case T_Q4_K: hipLaunchKernelGGL(gemm_q_kernel<GQ4K>, grid, block, 0, st, a, 0); break;
    case T_Q6_K: hipLaunchKernelGGL(gemm_q_kernel<GQ6K>, grid, block, 0, st, a, 0); break;
    default: hipLaunchKernelGGL(gemm_q_kernel<GQ80>, grid, block, 0, st, a, 0); break;
    }
    return hipGetLastError();
}

}  // namespace oi
