// gemm.hip -- batched projection for prefill on gfx950 matrix cores:
//   C[t][r] = sum_k f16(dequant(W)[r][k]) * X[t][k]     (f32 accumulate)
// for n tokens t at once (reference: the batched-prefill MMQ kernels
// qwen3_5/metal.odin:493-609 and gemm_harness/gemm_test.odin:97-135, 297-337,
// which stage both operands in half precision and accumulate in float).
// X is token-major f16 [n][K], C token-major f32 [n][M] (the transposes of the
// reference harness's B[K][N] and C[M][N]; same products).
//
// Work layout: a workgroup computes 128 rows x 64 tokens over a slice of K:
// wave w holds rows 16w .. 16w+15 in four v_mfma_f32_16x16x32_f16
// accumulators (16 tokens each) and walks the slice chunk by chunk (a chunk
// is one GEMV unit of 64 weights; two units = one super-block half for
// Q6_K); the chunk's activations are shared through LDS.  Every lane
// dequantizes the weights it feeds to
// the matrix cores straight from the plane layout (no LDS staging of W): for
// 16x16x32 the A operand of lane l is row l%16, k = 8(l/16) .. +7 of the
// 32-wide K step, and in the plane layout those are 8 consecutive bytes.
// Dequantization follows ggml/quant.odin exactly (separately rounded products,
// (d*sc)*q for Q6_K), then rounds to f16 (RNE), as the reference's staging.
//
// Operand layout of v_mfma_f32_16x16x32_f16 (per lane l, 8 halves each):
//   A[i][k]: i = l % 16, k = 8 (l / 16) + e;  B[k][j]: j = l % 16, k = 8 (l / 16) + e
//   D[i][j] (4 floats): j = l % 16, i = 4 (l / 16) + e.

#include <algorithm>

#include "device_common.h"

namespace oi {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int GM_WAVES = 8, GM_ROWS = 16 * GM_WAVES, GM_TOK = 64, GM_THREADS = GM_WAVES * WAVE;
constexpr int GM_PD = 4;  // weight chunks in the register ring (GM_PD - 1 in flight)

struct GemmArgs {
    DMat m;           // weights [M][K], device plane layout
    const uint16_t *x;  // [n][K] f16
    float *c;         // [n][M]
    int32_t n;
};

static __device__ __forceinline__ h8 cvt8(const float (&v)[8]) {
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; e++) r[e] = (_Float16)v[e];
    return r;
}

// ---- A operands of one chunk, per type --------------------------------------
// Each type has a raw load (the bytes a lane needs for one chunk, issued
// several chunks ahead) and a dequantization of those bytes into the chunk's
// A operands.
//
// Q4_K unit u (64 weights): K step 0 = low nibbles of bytes 0..31 (group 2p),
// step 1 = high nibbles (group 2p + 1); lane quarter q reads bytes 8q .. 8q+7
// (plane q/2, offset 8 (q%2)) and the super-block header.  ggml/quant.odin:178-209.
struct RawQ4K {
    u32x4 hdr;
    u32x2 b;
};
static __device__ __forceinline__ void raw_q4k(const DMat &m, int row, int u, int q, RawQ4K &r) {
    const size_t ui = (size_t)row * (m.cols >> 6) + u;
    r.hdr = *(const u32x4 *)(m.s + ((size_t)row * (m.cols >> 8) + (u >> 2)) * 16);
    r.b = *(const u32x2 *)(m.q + (q >> 1) * m.plane + ui * 16 + 8 * (q & 1));
}
static __device__ __forceinline__ void deq_q4k(const RawQ4K &r, int u, h8 *A) {
#pragma clang fp contract(off)
    const float d = h2f(r.hdr.x & 0xFFFFu), dmin = h2f(r.hdr.x >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(u & 3, r.hdr.y, r.hdr.z, r.hdr.w, sc0, m0, sc1, m1);
    const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
    const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
    float lo[8], hi[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const uint32_t by = ((e < 4 ? r.b.x : r.b.y) >> (8 * (e & 3))) & 0xFFu;
        lo[e] = d1 * (float)(by & 0xFu) - mm1;
        hi[e] = d2 * (float)(by >> 4) - mm2;
    }
    A[0] = cvt8(lo);
    A[1] = cvt8(hi);
}

// Q8_0 unit u: K step s covers block 2u + s; lane quarter q reads plane
// 2s + q/2 at offset 8 (q%2).  ggml/quant.odin:87-96.
struct RawQ80 {
    u32x2 b[2];
    uint32_t d;  // the two blocks' f16 scales
};
static __device__ __forceinline__ void raw_q80(const DMat &m, int row, int u, int q, RawQ80 &r) {
    const size_t ui = (size_t)row * (m.cols >> 6) + u;
    r.d = *(const uint32_t *)(m.d + (size_t)row * (m.cols >> 5) + 2 * u);
#pragma unroll
    for (int s = 0; s < 2; s++) r.b[s] = *(const u32x2 *)(m.q + (2 * s + (q >> 1)) * m.plane + ui * 16 + 8 * (q & 1));
}
static __device__ __forceinline__ void deq_q80(const RawQ80 &r, int, h8 *A) {
#pragma clang fp contract(off)
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const float d = h2f(s ? r.d >> 16 : r.d & 0xFFFFu);
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            v[e] = d * (float)(int8_t)(((e < 4 ? r.b[s].x : r.b[s].y) >> (8 * (e & 3))) & 0xFFu);
        A[s] = cvt8(v);
    }
}

// Q6_K chunk c = half h = c%2 of super-block sb = c/2 (units 4sb+2h, 4sb+2h+1):
// K step s is the 32 elements 128h + 32s + [0,32) (run s of both units); lane
// quarter q reads unit q/2 at byte offset 8 (q%2) of its ql-low, ql-high and
// qh planes; scale index 8h + q/2 + 2s.  ggml/quant.odin:212-247.
struct RawQ6K {
    u32x2 qa, qb, qh, scw;
    uint32_t d;
};
static __device__ __forceinline__ void raw_q6k(const DMat &m, int row, int c, int q, RawQ6K &r) {
    const int sb = c >> 1, h = c & 1, nsb = m.cols >> 8;
    const int u = 4 * sb + 2 * h + (q >> 1), off = 8 * (q & 1);
    const size_t ui = (size_t)row * (m.cols >> 6) + u, sbi = (size_t)row * nsb + sb;
    r.qa = *(const u32x2 *)(m.q + ui * 16 + off);
    r.qb = *(const u32x2 *)(m.q + m.plane + ui * 16 + off);
    r.qh = *(const u32x2 *)(m.q + 2 * m.plane + ui * 16 + off);
    r.scw = *(const u32x2 *)(m.s + sbi * 16 + 8 * h);
    r.d = m.d[sbi];
}
static __device__ __forceinline__ void deq_q6k(const RawQ6K &r, int, h8 *A, int q) {
#pragma clang fp contract(off)
    const float d = h2f(r.d);
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int is = (q >> 1) + 2 * s;
        const float ds = d * (float)(int8_t)(((is < 4 ? r.scw.x : r.scw.y) >> (8 * (is & 3))) & 0xFFu);
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t la = ((e < 4 ? r.qa.x : r.qa.y) >> (8 * (e & 3))) & 0xFFu;
            const uint32_t lb = ((e < 4 ? r.qb.x : r.qb.y) >> (8 * (e & 3))) & 0xFFu;
            const uint32_t hb = ((e < 4 ? r.qh.x : r.qh.y) >> (8 * (e & 3))) & 0xFFu;
            const uint32_t l4 = s == 0 ? (la & 0xF) : s == 1 ? (lb & 0xF) : s == 2 ? (la >> 4) : (lb >> 4);
            const int qv = (int)(l4 | (((hb >> (2 * s)) & 3u) << 4)) - 32;
            v[e] = ds * (float)qv;
        }
        A[s] = cvt8(v);
    }
}

template <int T> struct GemmType;
template <> struct GemmType<T_Q4_K> {
    using Raw = RawQ4K;
    static constexpr int SPC = 2;
    static __device__ void raw(const DMat &m, int row, int c, int q, Raw &r) { raw_q4k(m, row, c, q, r); }
    static __device__ void deq(const Raw &r, int c, int, h8 *A) { deq_q4k(r, c, A); }
};
template <> struct GemmType<T_Q8_0> {
    using Raw = RawQ80;
    static constexpr int SPC = 2;
    static __device__ void raw(const DMat &m, int row, int c, int q, Raw &r) { raw_q80(m, row, c, q, r); }
    static __device__ void deq(const Raw &r, int c, int, h8 *A) { deq_q80(r, c, A); }
};
template <> struct GemmType<T_Q6_K> {
    using Raw = RawQ6K;
    static constexpr int SPC = 4;
    static __device__ void raw(const DMat &m, int row, int c, int q, Raw &r) { raw_q6k(m, row, c, q, r); }
    static __device__ void deq(const Raw &r, int c, int q, h8 *A) { deq_q6k(r, c, A, q); }
};

// One workgroup: rows [128 bx, +128) (wave w: rows 16w .. 16w+15), tokens
// [64 by, +64), chunks [bz * cps, +cps) of K.  The 64 x KC activation chunk is
// staged in LDS once per workgroup (double-buffered, the next chunk's load in
// flight while this one is computed) and read by all 8 waves; each wave
// dequantizes its own rows.  With more than one K slice the partial products
// are added into c (zeroed by the launcher) with device-scope float atomics.
template <int T>
__global__ __launch_bounds__(GM_THREADS) void gemm_q_kernel(GemmArgs a, int cps, int split) {
    using G = GemmType<T>;
    constexpr int SPC = G::SPC;               // 32-wide K steps per chunk
    constexpr int KC = 32 * SPC;              // weights per chunk
    constexpr int XV = GM_TOK * KC / 8;       // 16-byte pieces of an activation chunk
    constexpr int XPT = XV / GM_THREADS;      // ... per thread
    __shared__ __attribute__((aligned(16))) u32x4 xs[2][XV];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int q = lane >> 4, li = lane & 15;
    const int M = a.m.rows, K = a.m.cols;
    const int row = min((int)blockIdx.x * GM_ROWS + 16 * wave + li, M - 1);  // rows past M: recomputed, not stored
    const int t0 = (int)blockIdx.y * GM_TOK;
    const int nchunk = K / KC;
    const int c0 = (int)blockIdx.z * cps, c1 = min(nchunk, c0 + cps);

    // piece p of a chunk: token p / (KC / 8), 8 activations at (p % (KC / 8)) * 8;
    // LDS slot of piece (token j, k-octet o): o * 64 + j (the B operand of lane
    // (j, q) for step s is octet 4s + q: consecutive lanes, consecutive slots)
    auto xfetch = [&](int c, u32x4 (&xr)[XPT]) {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int p = threadIdx.x + i * GM_THREADS, j = p / (KC / 8), o = p % (KC / 8);
            const int tok = min(t0 + j, a.n - 1);
            xr[i] = *(const u32x4 *)(a.x + (size_t)tok * K + (size_t)c * KC + 8 * o);
        }
    };
    auto xstore = [&](int buf, const u32x4 (&xr)[XPT]) {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int p = threadIdx.x + i * GM_THREADS, j = p / (KC / 8), o = p % (KC / 8);
            xs[buf][o * GM_TOK + j] = xr[i];
        }
    };

    f32x4v acc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) acc[t] = f32x4v{0.f, 0.f, 0.f, 0.f};
    // weights and activations GM_PD - 1 chunks ahead in register rings
    // (unconditional loads: chunks past the slice re-read its first, unused)
    typename G::Raw ring[GM_PD];
    u32x4 xr[GM_PD][XPT];
#pragma unroll
    for (int r = 0; r < GM_PD - 1; r++) {
        const int c = c0 + r < c1 ? c0 + r : c0;
        G::raw(a.m, row, c, q, ring[r]);
        xfetch(c, xr[r]);
    }
    for (int cb = c0; cb < c1; cb += GM_PD) {
#pragma unroll
        for (int r = 0; r < GM_PD; r++) {
            const int c = cb + r;
            if (c >= c1) break;
            const int cn = c + GM_PD - 1 < c1 ? c + GM_PD - 1 : c0, rn = (r + GM_PD - 1) % GM_PD;
            G::raw(a.m, row, cn, q, ring[rn]);
            xfetch(cn, xr[rn]);
            const int buf = (c - c0) & 1;
            xstore(buf, xr[r]);
            __syncthreads();  // chunk c staged; every wave is done with chunk c - 2's buffer
            h8 A[SPC];
            G::deq(ring[r], c, q, A);
#pragma unroll
            for (int s = 0; s < SPC; s++)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        A[s], __builtin_bit_cast(h8, xs[buf][(4 * s + q) * GM_TOK + 16 * t + li]), acc[t], 0, 0, 0);
        }
    }
    // D of token tile t: lane (j, g) holds rows 4g .. 4g+3 of column (token) j
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int tk = t0 + 16 * t + li;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int r = (int)blockIdx.x * GM_ROWS + 16 * wave + 4 * q + e;
            if (r < M && tk < a.n) {
                float *dst = a.c + (size_t)tk * M + r;
                if (split > 1) __hip_atomic_fetch_add(dst, acc[t][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else *dst = acc[t][e];
            }
        }
    }
}

bool gemm_supported(const DMat &m) {
    return (m.type == T_Q4_K || m.type == T_Q6_K) ? m.cols % 256 == 0 : m.type == T_Q8_0 && m.cols % 64 == 0;
}

// K is split so that about 192 workgroups run (each slice at least 4 chunks;
// measured best on 4096/12288 x 64 x 4096/12288); with more than one slice c is
// zeroed first and the slices add into it.
hipError_t launch_gemm(const DMat &m, const uint16_t *x, int32_t n, float *c, hipStream_t st) {
    if (!gemm_supported(m) || n <= 0) return hipErrorInvalidValue;
    GemmArgs a{m, x, c, n};
    const int kc = m.type == T_Q6_K ? 128 : 64, nchunk = m.cols / kc;
    const int tiles = ((m.rows + GM_ROWS - 1) / GM_ROWS) * ((n + GM_TOK - 1) / GM_TOK);
    int split = std::max(1, std::min((192 + tiles / 2) / tiles, nchunk / 4));  // ~192 workgroups (measured)
    const int cps = (nchunk + split - 1) / split;
    split = (nchunk + cps - 1) / cps;
    if (split > 1) {
        const hipError_t e = hipMemsetAsync(c, 0, (size_t)n * m.rows * 4, st);
        if (e != hipSuccess) return e;
    }
    dim3 grid((m.rows + GM_ROWS - 1) / GM_ROWS, (n + GM_TOK - 1) / GM_TOK, split), block(GM_THREADS);
    switch (m.type) {
    case T_Q4_K: hipLaunchKernelGGL(gemm_q_kernel<T_Q4_K>, grid, block, 0, st, a, cps, split); break;
    case T_Q6_K: hipLaunchKernelGGL(gemm_q_kernel<T_Q6_K>, grid, block, 0, st, a, cps, split); break;
    default: hipLaunchKernelGGL(gemm_q_kernel<T_Q8_0>, grid, block, 0, st, a, cps, split); break;
    }
    return hipGetLastError();
}

}  // namespace oi
