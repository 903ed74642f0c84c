// attn.hip -- split-L grouped-query decode attention over the f16 KV cache
// (reference: infer/forward.odin:87-115; f16 cache as infer/metal.odin:443-474).
//
// attn_kernel, grid (splits, n_kv_heads): a workgroup takes CH consecutive
// positions of one KV head and serves all G = n_heads / n_kv_heads query
// heads of the group, so each K/V row is read from HBM once per token (the
// reference re-reads it for every query head).  Per workgroup:
//   1. request this token's q (G heads), k, v, cos/sin and norm weights,
//      then its K and V tiles (16 B per lane, coalesced); every load is
//      unconditional (rows past the range re-read a valid row and are zeroed
//      later), so the compiler waits for the small loads alone while the
//      tiles stream,
//   2. RMSNorm + RoPE the G query heads (and, in the split that holds `pos`,
//      the new key; K/V[pos] are rounded to f16 and stored),
//   3. stage K (rows padded against bank conflicts) and V in LDS,
//   4. one wave per query head, with no workgroup barrier: scores with lane l
//      taking position l (the whole dot product of its K row), divided by
//      sqrt(hd) (infer/forward.odin:98); split max / exp-sum by wave reductions;
//      o = sum_t p v_t with 2 dims per lane and p read from the wave's LDS row,
//   5. write (o, m, l) to the partial buffer.
// attn_combine_kernel merges the splits of each query head with
// exp(m_s - M) weights; the kernel boundary orders the partial writes before
// the reads, so no fences or atomics are needed.  (Merging in the last
// arriving split instead costs a store-completion wait, an atomic and the
// partial reads in series, which measured slower than the kernel boundary.)
// The current position is used from LDS, so no workgroup reads a cache
// entry written in this launch.

#include <algorithm>

#include "device_common.h"

namespace oi {

// threads of an attn_kernel workgroup: one wave per query head of the group
// (at least 4 waves), so no wave computes two heads in series
static constexpr int attn_threads(int G) { return G > 4 ? G * WAVE : WG; }

template <int HD>
struct AttnShape {
    static constexpr int CH = 64;                     // positions per workgroup (one per lane)
    static constexpr int KPAD = HD + 8;               // LDS row stride of K, in halves
    static constexpr int CPR = HD / 8;                // 16-byte chunks per row
    static constexpr int DPW = HD / 4;                // score dimensions per wave
    static constexpr int DPL = HD / WAVE;             // o dimensions per lane
    static constexpr int PPL = CH / WAVE;             // score positions per lane
};
constexpr int ATTN_MAX_SPLITS = 1024;

// head_dim 128 kernel (attn128_kernel below): 16 waves, splits of at most
// A128_CHMAX positions, their length 16 * ceil(ceil(n / max_splits) / 16)
constexpr int A128_NT = 1024, A128_NW = A128_NT / WAVE;
constexpr int A128_CHMAX = 256;                     // positions per split at most (a tile of 16 per wave)

static __device__ __forceinline__ int a128_split_len(int n, int max_splits) {
    const int per = (n + max_splits - 1) / max_splits;
    return (per + 15) & ~15;
}


template <int HD, int G>
__global__ __launch_bounds__(attn_threads(G)) void attn_kernel(AttnArgs a) {
    using S = AttnShape<HD>;
    constexpr int NT = attn_threads(G), NLD = S::CH * S::CPR / NT;  // threads; tile loads per thread per tensor
    __shared__ __attribute__((aligned(16))) uint16_t ks[S::CH * S::KPAD];
    __shared__ __attribute__((aligned(16))) uint16_t vs[S::CH * HD];
    __shared__ __attribute__((aligned(16))) float qr[G][HD];
    __shared__ float kp[HD], vp[HD], qn[HD], kn[HD];
    __shared__ __attribute__((aligned(16))) float sp[1][G][S::CH];  // p of each head (its wave's row)
    __shared__ float nrm[G + 1];
    __shared__ float2 csl[HD / 2];

    const int split = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int pos = a.state[ST_POS];
    const int t0 = split * S::CH;
    if (t0 > pos) return;
    const int t1 = min(t0 + S::CH, pos + 1), n = t1 - t0;
    uint16_t *kc = a.kc + (size_t)kvh * a.seq_len * HD;
    uint16_t *vc = a.vc + (size_t)kvh * a.seq_len * HD;
    const bool has_pos = pos < t1;

    // 1. small loads first (vector loads return in order), then the tiles
    constexpr int QPT = (G * HD + NT - 1) / NT;
    float qreg[QPT];
#pragma unroll
    for (int i = 0; i < QPT; i++) qreg[i] = a.q[(size_t)kvh * G * HD + min(tid + i * NT, G * HD - 1)];
    const int hi = min(tid, HD - 1);
    const float kraw = a.k[(size_t)kvh * HD + hi], vraw = a.v[(size_t)kvh * HD + hi];
    const float2 csr = a.rope_cs[(size_t)pos * (HD / 2) + min(tid, HD / 2 - 1)];
    const float qnr = a.q_norm[hi], knr = a.k_norm[hi];
    u32x4 kr[NLD], vr[NLD];
#pragma unroll
    for (int j = 0; j < NLD; j++) {
        const int c = tid + j * NT, tl = min(c / S::CPR, n - 1), ch = c % S::CPR;
        kr[j] = ldg_nt((const u32x4 *)(kc + (size_t)(t0 + tl) * HD) + ch);
        vr[j] = ldg_nt((const u32x4 *)(vc + (size_t)(t0 + tl) * HD) + ch);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. RMSNorm + RoPE of the G query heads (and of k at pos): infer/ops.odin:7-19,
    //    infer/forward.odin:57-85; cos/sin come from the host-built table
#pragma unroll
    for (int i = 0; i < QPT; i++) {
        const int idx = tid + i * NT;
        if (idx < G * HD) qr[idx / HD][idx % HD] = qreg[i];
    }
    if (tid < HD) {
        kp[tid] = kraw;
        vp[tid] = vraw;
        qn[tid] = qnr;
        kn[tid] = knr;
    }
    if (tid < HD / 2) csl[tid] = csr;
    __syncthreads();
    const int nvec = G + (has_pos ? 1 : 0);
    for (int g = wave; g < nvec; g += NT / WAVE) {
        const float *src = g < G ? qr[g] : kp;
        float ss = 0.f;
        for (int i = lane; i < HD; i += WAVE) ss += src[i] * src[i];
        ss = wave_sum(ss);
        if (lane == 0) nrm[g] = 1.0f / sqrtf(ss / (float)HD + a.eps);
    }
    __syncthreads();
    for (int idx = tid; idx < nvec * (HD / 2); idx += NT) {
#pragma clang fp contract(off)
        const int g = idx / (HD / 2), i = idx % (HD / 2);
        float *v = g < G ? qr[g] : kp;
        const float *w = g < G ? qn : kn;
        const float s = nrm[g];
        const float x = w[i] * (s * v[i]);
        const float y = w[i + HD / 2] * (s * v[i + HD / 2]);
        const float c = csl[i].x, sn = csl[i].y;
        v[i] = x * c - y * sn;
        v[i + HD / 2] = x * sn + y * c;
    }

    // 3. stage the tiles in LDS (rows at or past n are zero; row pos-t0 is set below)
#pragma unroll
    for (int j = 0; j < NLD; j++) {
        const int c = tid + j * NT, tl = c / S::CPR, ch = c % S::CPR;
        const bool ok = tl < n && t0 + tl != pos;
        const u32x4 z = {0u, 0u, 0u, 0u};
        *(u32x4 *)(ks + tl * S::KPAD + ch * 8) = ok ? kr[j] : z;
        *(u32x4 *)(vs + tl * HD + ch * 8) = ok ? vr[j] : z;
    }
    __syncthreads();
    if (has_pos) {
        const int tl = pos - t0;
        for (int i = tid; i < HD; i += NT) {
            const uint16_t kb = f2h(kp[i]), vb = f2h(vp[i]);
            kc[(size_t)pos * HD + i] = kb;
            vc[(size_t)pos * HD + i] = vb;
            ks[tl * S::KPAD + i] = kb;
            vs[tl * HD + i] = vb;
        }
        __syncthreads();
    }

    // 4-6. one wave per query head, no workgroup barrier: scores with lane =
    // position (each lane the whole dot product of its row), split max and
    // exp-sum by wave reductions (infer/ops.odin:21-37), p through this wave's LDS
    // row, o = sum_t p(t) v(t) with DPL dimensions per lane, then the split's
    // (o, m, l).  Score = q.k / sqrt(hd) (infer/forward.odin:98 divides).
    const float div = sqrtf((float)HD);
    const int stride = HD + 2;
    for (int g = wave; g < G; g += NT / WAVE) {
        float sc[S::PPL], m = -INFINITY;
#pragma unroll
        for (int p = 0; p < S::PPL; p++) {
            const int t = lane + WAVE * p;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};  // four chains over the 8-dimension chunks
#pragma unroll
            for (int c = 0; c < HD / 8; c++) {
                const u32x4 w = *(const u32x4 *)(ks + t * S::KPAD + 8 * c);
                const float4 q0 = *(const float4 *)&qr[g][8 * c];
                const float4 q1 = *(const float4 *)&qr[g][8 * c + 4];
                acc[c & 3] += q0.x * h2f(w.x & 0xFFFFu) + q0.y * h2f(w.x >> 16) + q0.z * h2f(w.y & 0xFFFFu) +
                              q0.w * h2f(w.y >> 16) + q1.x * h2f(w.z & 0xFFFFu) + q1.y * h2f(w.z >> 16) +
                              q1.z * h2f(w.w & 0xFFFFu) + q1.w * h2f(w.w >> 16);
            }
            sc[p] = t < n ? ((acc[0] + acc[1]) + (acc[2] + acc[3])) / div : -INFINITY;
            m = fmaxf(m, sc[p]);
        }
        m = wave_max_all(m);
        float l = 0.f;
#pragma unroll
        for (int p = 0; p < S::PPL; p++) {
            const int t = lane + WAVE * p;
            const float e = t < n ? expf(sc[p] - m) : 0.f;
            sp[0][g][t] = e;  // this wave's row only: DS operations of one wave complete in order
            l += e;
        }
        l = wave_sum(l);
        __builtin_amdgcn_wave_barrier();
        float acc[4][S::DPL];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < S::DPL; e++) acc[j][e] = 0.f;
#pragma unroll 4
        for (int t4 = 0; t4 < S::CH; t4 += 4) {
            const float4 p4 = *(const float4 *)&sp[0][g][t4];  // rows past n hold p = 0 and zero V
            const float pw[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float vv[S::DPL];
                if (S::DPL == 2) {
                    const uint32_t w = *(const uint32_t *)(vs + (t4 + j) * HD + 2 * lane);
                    vv[0] = h2f(w & 0xFFFFu);
                    vv[S::DPL - 1] = h2f(w >> 16);
                } else {
                    const u32x2 w = *(const u32x2 *)(vs + (t4 + j) * HD + S::DPL * lane);
                    const uint32_t ws[2] = {w.x, w.y};
#pragma unroll
                    for (int e = 0; e < S::DPL; e++) vv[e] = h2f((ws[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
                }
#pragma unroll
                for (int e = 0; e < S::DPL; e++) acc[j][e] += pw[j] * vv[e];
            }
        }
        float *pp = a.part + ((size_t)(kvh * G + g) * a.max_splits + split) * stride;
#pragma unroll
        for (int e = 0; e < S::DPL; e++)
            pp[S::DPL * lane + e] = (acc[0][e] + acc[1][e]) + (acc[2][e] + acc[3][e]);
        if (lane == 0) {
            pp[HD] = m;
            pp[HD + 1] = l;
        }
    }
}

// O_h = sum_s exp(m_s - M) o_s / sum_s exp(m_s - M) l_s  for one query head and
// 64 of its dimensions; the 4 waves take every 4th split.  The o values of
// the first 4 CMB_PF splits are requested together with the (m, l) pairs (one
// memory round trip instead of two); longer caches read the rest afterwards.
constexpr int CMB_PF = 20;
template <int HD>
__global__ __launch_bounds__(WG) void attn_combine_kernel(AttnArgs a) {
    using S = AttnShape<HD>;
    __shared__ float wm[ATTN_MAX_SPLITS], wl[ATTN_MAX_SPLITS];
    __shared__ float ored[WG / WAVE][WAVE];
    __shared__ float Ls;
    const int h = blockIdx.x, i = blockIdx.y * WAVE + (threadIdx.x & (WAVE - 1));
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int pos = a.state[ST_POS];
    // fixed splits of CH positions, or (a.chunk == 0) splits sized from pos
    const int nsplit = a.chunk > 0 ? pos / S::CH + 1 : (pos + a128_split_len(pos + 1, a.max_splits)) /
                                                           a128_split_len(pos + 1, a.max_splits);
    const int stride = HD + 2;
    const float *pb = a.part + (size_t)h * a.max_splits * stride;
    float ov[CMB_PF];
#pragma unroll
    for (int k = 0; k < CMB_PF; k++) {
        const int s = wave + (WG / WAVE) * k;
        ov[k] = s < nsplit ? pb[(size_t)s * stride + i] : 0.f;
    }
    for (int s = tid; s < nsplit; s += WG) {
        wm[s] = pb[(size_t)s * stride + HD];
        wl[s] = pb[(size_t)s * stride + HD + 1];
    }
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
        for (int s = lane; s < nsplit; s += WAVE) M = fmaxf(M, wm[s]);
        M = wave_max_all(M);
        float L = 0.f;
        for (int s = lane; s < nsplit; s += WAVE) {
            const float f = expf(wm[s] - M);
            wm[s] = f;
            L += f * wl[s];
        }
        L = wave_sum(L);
        if (lane == 0) Ls = L;
    }
    __syncthreads();
    float O = 0.f;
#pragma unroll
    for (int k = 0; k < CMB_PF; k++) {
        const int s = wave + (WG / WAVE) * k;
        if (s < nsplit) O += wm[s] * ov[k];
    }
#pragma unroll 8
    for (int s = wave + (WG / WAVE) * CMB_PF; s < nsplit; s += WG / WAVE) O += wm[s] * pb[(size_t)s * stride + i];
    ored[wave][lane] = O;
    __syncthreads();
    if (wave == 0) a.out[(size_t)h * HD + i] = ((ored[0][lane] + ored[1][lane]) + (ored[2][lane] + ored[3][lane])) / Ls;
}

// ---------------------------------------------------------------------------
// head_dim 128: splits sized from pos at run time (a.chunk == 0).
//
// attn128_kernel, grid (max_splits, n_kv_heads), 16 waves: the n = pos + 1
// positions are cut into splits of ch = 16 * ceil(ceil(n / max_splits) / 16)
// positions, max_splits chosen by the host so that about one workgroup per
// CU is busy at every cache length.  A split is at most 16 tiles of 16 keys;
// wave w takes tile w and works alone until the last step:
//   1. requests this token's q (G heads), k, v, cos/sin and norms, then its
//      tiles' K straight into the matrix-core operand layout (lane (r, g)
//      holds dims 32c + 8g .. +7 of key r of the tile: four 16-byte pieces
//      per key, no LDS staging) and its tiles' V rows (lane l: dims 2l, 2l+1
//      of each key, one 4-byte piece per key, 256 contiguous bytes per key);
//   2. the workgroup RMSNorms and RoPEs the G query heads (and, in the split
//      holding pos, the new key, whose K/V are rounded to f16, stored to the
//      cache and put in place of the stale rows the tiles read), as the
//      token's operations of infer/forward.odin:57-85;
//   3. scores S^T[key][col] = K Q^T on v_mfma_f32_16x16x32_f16: column h < G
//      is head h's q rounded to f16, column G + h its remainder q - f16(q)
//      (so q keeps about 22 bits; K is exact f16, products exact, sums f32);
//      the two columns are added (a DPP row shift), divided by sqrt(hd)
//      (infer/forward.odin:98);
//   4. the wave's softmax over its keys (max, exp, sum: infer/ops.odin:21-37) and
//      o = sum_t p_t v_t for its keys, 2 dimensions per lane, all heads;
//   5. the waves' (o, m, l) merged through LDS with exp(m_w - M) weights
//      into the split's (o, m, l), which attn_combine_kernel merges across
//      splits.
typedef _Float16 a128_h8 __attribute__((ext_vector_type(8)));
typedef float a128_f4 __attribute__((ext_vector_type(4)));
constexpr int A128_TPW = A128_CHMAX / 16 / A128_NW;  // 16-key tiles per wave at most
static_assert(A128_TPW * 16 * A128_NW == A128_CHMAX, "whole tiles per wave");

template <int G>
__global__ __launch_bounds__(A128_NT) void attn128_kernel(AttnArgs a) {
    constexpr int HD = 128;
    static_assert(2 * G <= 16, "hi and lo columns of every head fit one 16-column tile");
    static_assert(A128_TPW == 1, "one tile per wave");
    __shared__ __attribute__((aligned(16))) float qr[G][HD];
    __shared__ __attribute__((aligned(16))) float wp[A128_NW][G][16];  // each wave's p
    __shared__ __attribute__((aligned(16))) float red[A128_NW][G][HD];  // each wave's o
    __shared__ float wm[A128_NW][G], wl[A128_NW][G];
    __shared__ __attribute__((aligned(16))) float kp[HD], vp[HD], qn[HD], kn[HD];
    __shared__ float nrm[G + 1];
    __shared__ __attribute__((aligned(16))) float2 csl[HD / 2];

    const int split = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & (WAVE - 1), wave = tid / WAVE, r16 = lane & 15, g4 = lane >> 4;
    const int pos = a.state[ST_POS];
    const int n_all = pos + 1;
    const int ch = a128_split_len(n_all, a.max_splits);
    const int t0 = split * ch;
    if (t0 >= n_all) return;
    const int t1 = min(t0 + ch, n_all), n = t1 - t0;
    const int ntile = (n + 15) >> 4;
    uint16_t *kc = a.kc + (size_t)kvh * a.seq_len * HD;
    uint16_t *vc = a.vc + (size_t)kvh * a.seq_len * HD;
    const bool has_pos = pos < t1;

    // 1. the small loads (16 bytes per thread, by the threads that need them),
    //    all arrived before any tile is requested: issued together with every
    //    workgroup's tiles they queue behind them (3-4 us instead of ~1)
    constexpr int NQ4 = G * HD / 4;
    float4 q4 = make_float4(0.f, 0.f, 0.f, 0.f), k4 = q4, v4 = q4, qn4 = q4, kn4 = q4, cs4 = q4;
    if (tid < NQ4) q4 = ((const float4 *)(a.q + (size_t)kvh * G * HD))[tid];
    if (tid < HD / 4) {
        k4 = ((const float4 *)(a.k + (size_t)kvh * HD))[tid];
        v4 = ((const float4 *)(a.v + (size_t)kvh * HD))[tid];
        qn4 = ((const float4 *)a.q_norm)[tid];
        kn4 = ((const float4 *)a.k_norm)[tid];
        cs4 = ((const float4 *)(a.rope_cs + (size_t)pos * (HD / 2)))[tid];
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    // the tile: K straight into the operand layout (lane (r16, g4): dims
    // 32c + 8g4 .. +7 of key r16), V as 8-byte pieces (lane (dq, kh): dims
    // 4dq .. 4dq+3 of keys 8kh .. 8kh+7); a wave past the split's tiles reads
    // row t0 for every lane (unconditional loads keep the compiler's count)
    const int kt = wave, dq = lane & 31, kh = lane >> 5;
    u32x4 kr[4] = {};
    u32x2 vr[8] = {};
    if (kt < ntile) {  // wave-uniform: a wave past the split's tiles requests nothing
        const int row = t0 + min(16 * kt + r16, n - 1);
#pragma unroll
        for (int c = 0; c < 4; c++) kr[c] = ldg_nt((const u32x4 *)(kc + (size_t)row * HD + 32 * c + 8 * g4));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int rv = t0 + min(16 * kt + 8 * kh + k, n - 1);
            vr[k] = ldg_nt((const u32x2 *)(vc + (size_t)rv * HD + 4 * dq));
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. RMSNorm + RoPE of the query heads and of k at pos (infer/ops.odin:7-19,
    //    infer/forward.odin:57-85; cos/sin from the host-built table)
    if (tid < NQ4) *(float4 *)&qr[tid / (HD / 4)][4 * (tid % (HD / 4))] = q4;
    if (tid < HD / 4) {
        *(float4 *)&kp[4 * tid] = k4;
        *(float4 *)&vp[4 * tid] = v4;
        *(float4 *)&qn[4 * tid] = qn4;
        *(float4 *)&kn[4 * tid] = kn4;
        *(float4 *)&csl[2 * tid] = cs4;
    }
    __syncthreads();
    const int nvec = G + (has_pos ? 1 : 0);
    for (int g = wave; g < nvec; g += A128_NW) {
        const float *src = g < G ? qr[g] : kp;
        float ss = 0.f;
        for (int i = lane; i < HD; i += WAVE) ss += src[i] * src[i];
        ss = wave_sum(ss);
        if (lane == 0) nrm[g] = 1.0f / sqrtf(ss / (float)HD + a.eps);
    }
    __syncthreads();
    for (int idx = tid; idx < nvec * (HD / 2); idx += A128_NT) {
#pragma clang fp contract(off)
        const int g = idx / (HD / 2), i = idx % (HD / 2);
        float *v = g < G ? qr[g] : kp;
        const float *w = g < G ? qn : kn;
        const float s = nrm[g];
        const float x = w[i] * (s * v[i]);
        const float y = w[i + HD / 2] * (s * v[i + HD / 2]);
        const float c = csl[i].x, sn = csl[i].y;
        v[i] = x * c - y * sn;
        v[i + HD / 2] = x * sn + y * c;
    }
    __syncthreads();
    if (has_pos && tid < HD) {  // the new K/V row of the cache (read by later tokens)
        kc[(size_t)pos * HD + tid] = f2h(kp[tid]);
        vc[(size_t)pos * HD + tid] = f2h(vp[tid]);
    }

    // B operand, built once per workgroup: column r16 = head r16 (f16 of q)
    // or head r16 - G (its remainder q - f16(q)), zero past 2G; lane (r16, g4)
    // of every wave reads dims 32c + 8g4 .. +7 of chunk c
    __shared__ __attribute__((aligned(16))) u32x4 qbl[4][WAVE];
    if (tid < 4 * WAVE) {
        const int c = tid / WAVE, l = tid % WAVE, col = l & 15, gg = l >> 4;
        const int hq = col < G ? col : col - G;
        uint32_t w[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; e2++) {
            uint32_t hw[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float v = col < 2 * G ? qr[hq][32 * c + 8 * gg + 2 * e2 + j] : 0.f;
                const _Float16 h = (_Float16)v;
                const _Float16 r = col < G ? h : (_Float16)(v - (float)h);
                hw[j] = (uint32_t)__builtin_bit_cast(uint16_t, r);
            }
            w[e2] = hw[0] | (hw[1] << 16);
        }
        qbl[c][l] = u32x4{w[0], w[1], w[2], w[3]};
    }
    __syncthreads();
    a128_h8 qb[4];
#pragma unroll
    for (int c = 0; c < 4; c++) qb[c] = __builtin_bit_cast(a128_h8, qbl[c][lane]);

    // 3-4. this wave's tile: scores, softmax, o
    const float div = sqrtf((float)HD);
    float sc[4];
    float m = -INFINITY;
    {
        if (has_pos && kt < ntile && (pos - t0) >> 4 == kt && (pos - t0) % 16 == r16) {
            // this lane's key is pos: its K is the new one, not the stale cache row
#pragma unroll
            for (int c = 0; c < 4; c++) {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    w[e] = (uint32_t)f2h(kp[32 * c + 8 * g4 + 2 * e]) |
                           ((uint32_t)f2h(kp[32 * c + 8 * g4 + 2 * e + 1]) << 16);
                kr[c] = u32x4{w[0], w[1], w[2], w[3]};
            }
        }
        a128_f4 acc = a128_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; c++)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(a128_h8, kr[c]), qb[c], acc, 0, 0, 0);
        // the result's elements as plain registers: hipcc (ROCm 7.2) emitted
        // every DPP move below from element 0 when it read acc[e] directly
        float av[4] = {acc[0], acc[1], acc[2], acc[3]};
#pragma unroll
        for (int e = 0; e < 4; e++) asm volatile("" : "+v"(av[e]));
#pragma unroll
        for (int e = 0; e < 4; e++) {
            // lane (h, g4) for h < G: head h's score of key 16 kt + 4 g4 + e
            // (the remainder column G + h comes from lane h + G: row_shl:G)
            const float lo = __builtin_bit_cast(
                float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, av[e]), 0x100 + G, 0xF, 0xF, false));
            const int t = 16 * kt + 4 * g4 + e;
            sc[e] = kt < ntile && t < n ? (av[e] + lo) / div : -INFINITY;
            m = fmaxf(m, sc[e]);
        }
    }
    m = fmaxf(m, __shfl_xor(m, 16, WAVE));
    m = fmaxf(m, __shfl_xor(m, 32, WAVE));
    float l = 0.f;
    {
        float pe[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            pe[e] = m == -INFINITY ? 0.f : expf(sc[e] - m);
            l += pe[e];
        }
        if (r16 < G) *(float4 *)&wp[wave][r16][4 * g4] = make_float4(pe[0], pe[1], pe[2], pe[3]);
    }
    l += __shfl_xor(l, 16, WAVE);
    l += __shfl_xor(l, 32, WAVE);
    if (lane < G) {
        wm[wave][lane] = m;
        wl[wave][lane] = l;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's p rows are in LDS
    __builtin_amdgcn_wave_barrier();
    // o over the tile's keys 8kh .. 8kh+7 for dims 4dq .. 4dq+3, then the two
    // halves of the keys added (lanes dq and dq + 32)
    float o[G][4];
#pragma unroll
    for (int h = 0; h < G; h++) o[h][0] = o[h][1] = o[h][2] = o[h][3] = 0.f;
    if (kt < ntile) {
        const int kp0 = has_pos && (pos - t0) >> 4 == kt ? (pos - t0) & 15 : -1;
#pragma unroll
        for (int k4 = 0; k4 < 8; k4 += 4) {
            float4 p4[G];
#pragma unroll
            for (int h = 0; h < G; h++) p4[h] = *(const float4 *)&wp[wave][h][8 * kh + k4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int k = k4 + j;
                u32x2 w = vr[k];
                if (8 * kh + k == kp0)  // key pos: the new V, not the stale cache row
                    w = u32x2{(uint32_t)f2h(vp[4 * dq]) | ((uint32_t)f2h(vp[4 * dq + 1]) << 16),
                              (uint32_t)f2h(vp[4 * dq + 2]) | ((uint32_t)f2h(vp[4 * dq + 3]) << 16)};
                const float v0 = h2f(w.x & 0xFFFFu), v1 = h2f(w.x >> 16), v2 = h2f(w.y & 0xFFFFu),
                            v3 = h2f(w.y >> 16);
#pragma unroll
                for (int h = 0; h < G; h++) {
                    const float pk = j == 0 ? p4[h].x : j == 1 ? p4[h].y : j == 2 ? p4[h].z : p4[h].w;
                    o[h][0] += pk * v0;
                    o[h][1] += pk * v1;
                    o[h][2] += pk * v2;
                    o[h][3] += pk * v3;
                }
            }
        }
    }
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int j = 0; j < 4; j++) o[h][j] += __shfl_xor(o[h][j], 32, WAVE);
    if (kh == 0) {
#pragma unroll
        for (int h = 0; h < G; h++) *(float4 *)&red[wave][h][4 * dq] = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
    }
    __syncthreads();

    // 5. merge the waves (a wave without keys has m = -inf, l = 0, o = 0):
    //    the weights exp(m_w - M) once per (wave, head), then the sums
    __shared__ float wf[A128_NW][G], hM[G], hL[G];
    if (tid < G * A128_NW) {
        const int h = tid / A128_NW, w = tid % A128_NW;
        float M = -INFINITY;
#pragma unroll
        for (int x = 0; x < A128_NW; x++) M = fmaxf(M, wm[x][h]);
        const float f = wm[w][h] == -INFINITY ? 0.f : expf(wm[w][h] - M);
        wf[w][h] = f;
        if (w == 0) {
            float L = 0.f;
#pragma unroll
            for (int x = 0; x < A128_NW; x++) L += (wm[x][h] == -INFINITY ? 0.f : expf(wm[x][h] - M)) * wl[x][h];
            hM[h] = M;
            hL[h] = L;
        }
    }
    __syncthreads();
    const int stride = HD + 2;
    for (int idx = tid; idx < G * HD; idx += A128_NT) {
        const int h = idx / HD, d = idx % HD;
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < A128_NW; w++) acc += wf[w][h] * red[w][h][d];
        float *pp = a.part + ((size_t)(kvh * G + h) * a.max_splits + split) * stride;
        pp[d] = acc;
        if (d == 0) {
            pp[HD] = hM[h];
            pp[HD + 1] = hL[h];
        }
    }
}

template <int HD>
static hipError_t launch_attn_hd(const AttnArgs &a, int G, hipStream_t st) {
    dim3 grid(a.max_splits, a.n_kv_heads);
    switch (G) {
    case 1: hipLaunchKernelGGL((attn_kernel<HD, 1>), grid, dim3(attn_threads(1)), 0, st, a); break;
    case 2: hipLaunchKernelGGL((attn_kernel<HD, 2>), grid, dim3(attn_threads(2)), 0, st, a); break;
    case 4: hipLaunchKernelGGL((attn_kernel<HD, 4>), grid, dim3(attn_threads(4)), 0, st, a); break;
    case 8: hipLaunchKernelGGL((attn_kernel<HD, 8>), grid, dim3(attn_threads(8)), 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(a.n_heads, HD / WAVE), dim3(WG), 0, st, a);
    return hipGetLastError();
}

static hipError_t launch_attn128(const AttnArgs &a, int G, hipStream_t st) {
    dim3 grid(a.max_splits, a.n_kv_heads), block(A128_NT);
    switch (G) {
    case 1: hipLaunchKernelGGL((attn128_kernel<1>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((attn128_kernel<2>), grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL((attn128_kernel<4>), grid, block, 0, st, a); break;
    case 8: hipLaunchKernelGGL((attn128_kernel<8>), grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((attn_combine_kernel<128>), dim3(a.n_heads, 128 / WAVE), dim3(WG), 0, st, a);
    return hipGetLastError();
}

// Split plan: head_dim 128 sizes its splits from pos (chunk 0) with enough
// splits that n_kv_heads x splits covers the CUs (256) and no split exceeds
// A128_CHMAX positions at seq_len; head_dim 256 (and 128 with `fixed`, the
// lane-per-position kernel) keeps splits of 64.
int attn_plan(int head_dim, int n_kv_heads, int seq_len, int *chunk, bool fixed) {
    if (head_dim == 128 && !fixed) {
        *chunk = 0;
        const int by_cus = (256 + n_kv_heads - 1) / std::max(n_kv_heads, 1);
        return std::max(by_cus, (seq_len + A128_CHMAX - 1) / A128_CHMAX);
    }
    *chunk = attn_chunk(head_dim);
    return (seq_len + *chunk - 1) / *chunk;
}
int attn_chunk(int head_dim) { return head_dim == 256 ? AttnShape<256>::CH : AttnShape<128>::CH; }
int attn_max_splits() { return ATTN_MAX_SPLITS; }

hipError_t launch_attn(const AttnArgs &a, int head_dim, hipStream_t st) {
    const int G = a.n_heads / a.n_kv_heads;
    if (a.max_splits > ATTN_MAX_SPLITS || a.max_splits < 1) return hipErrorInvalidValue;
    if (head_dim == 128 && a.chunk == 0) {
        // every split of the plan must fit the LDS tile at seq_len
        if ((long)a.max_splits * A128_CHMAX < a.seq_len) return hipErrorInvalidValue;
        return launch_attn128(a, G, st);
    }
    if (a.chunk != attn_chunk(head_dim)) return hipErrorInvalidValue;
    if (head_dim == 128) return launch_attn_hd<128>(a, G, st);
    if (head_dim == 256) return launch_attn_hd<256>(a, G, st);
    return hipErrorInvalidValue;
}

}  // namespace oi
