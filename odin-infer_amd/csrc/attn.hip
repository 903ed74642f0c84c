// attn.hip -- split-L grouped-query decode attention over the f16 KV cache
// (reference: infer/forward.odin:117-175; f16 cache as infer/metal.odin:443-474).
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
//      sqrt(hd) (forward.odin:158); split max / exp-sum by wave reductions;
//      o = sum_t p v_t with 2 dims per lane and p read from the wave's LDS row,
//   5. write (o, m, l) to the partial buffer.
// attn_combine_kernel merges the splits of each query head with
// exp(m_s - M) weights; the kernel boundary orders the partial writes before
// the reads, so no fences or atomics are needed.  (Merging in the last
// arriving split instead costs a store-completion wait, an atomic and the
// partial reads in series, which measured slower than the kernel boundary.)
// The current position is used from LDS, so no workgroup reads a cache
// entry written in this launch.

#include "device_common.h"

namespace oi {

template <int HD>
struct AttnShape {
    static constexpr int CH = 64;                     // positions per workgroup (one per lane)
    static constexpr int KPAD = HD + 8;               // LDS row stride of K, in halves
    static constexpr int CPR = HD / 8;                // 16-byte chunks per row
    static constexpr int NLD = CH * CPR / WG;         // loads per thread per tensor
    static constexpr int DPW = HD / 4;                // score dimensions per wave
    static constexpr int DPL = HD / WAVE;             // o dimensions per lane
    static constexpr int PPL = CH / WAVE;             // score positions per lane
};
constexpr int ATTN_MAX_SPLITS = 1024;


template <int HD, int G>
__global__ __launch_bounds__(WG) void attn_kernel(AttnArgs a) {
    using S = AttnShape<HD>;
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
    constexpr int QPT = (G * HD + WG - 1) / WG;
    float qreg[QPT];
#pragma unroll
    for (int i = 0; i < QPT; i++) qreg[i] = a.q[(size_t)kvh * G * HD + min(tid + i * WG, G * HD - 1)];
    const int hi = min(tid, HD - 1);
    const float kraw = a.k[(size_t)kvh * HD + hi], vraw = a.v[(size_t)kvh * HD + hi];
    const float2 csr = a.rope_cs[(size_t)pos * (HD / 2) + min(tid, HD / 2 - 1)];
    const float qnr = a.q_norm[hi], knr = a.k_norm[hi];
    u32x4 kr[S::NLD], vr[S::NLD];
#pragma unroll
    for (int j = 0; j < S::NLD; j++) {
        const int c = tid + j * WG, tl = min(c / S::CPR, n - 1), ch = c % S::CPR;
        kr[j] = ldg_nt((const u32x4 *)(kc + (size_t)(t0 + tl) * HD) + ch);
        vr[j] = ldg_nt((const u32x4 *)(vc + (size_t)(t0 + tl) * HD) + ch);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. RMSNorm + RoPE of the G query heads (and of k at pos): ops.odin:7-19,
    //    forward.odin:117-145; cos/sin come from the host-built table
#pragma unroll
    for (int i = 0; i < QPT; i++) {
        const int idx = tid + i * WG;
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
    for (int g = wave; g < nvec; g += WG / WAVE) {
        const float *src = g < G ? qr[g] : kp;
        float ss = 0.f;
        for (int i = lane; i < HD; i += WAVE) ss += src[i] * src[i];
        ss = wave_sum(ss);
        if (lane == 0) nrm[g] = 1.0f / sqrtf(ss / (float)HD + a.eps);
    }
    __syncthreads();
    for (int idx = tid; idx < nvec * (HD / 2); idx += WG) {
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
    for (int j = 0; j < S::NLD; j++) {
        const int c = tid + j * WG, tl = c / S::CPR, ch = c % S::CPR;
        const bool ok = tl < n && t0 + tl != pos;
        const u32x4 z = {0u, 0u, 0u, 0u};
        *(u32x4 *)(ks + tl * S::KPAD + ch * 8) = ok ? kr[j] : z;
        *(u32x4 *)(vs + tl * HD + ch * 8) = ok ? vr[j] : z;
    }
    __syncthreads();
    if (has_pos) {
        const int tl = pos - t0;
        for (int i = tid; i < HD; i += WG) {
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
    // exp-sum by wave reductions (ops.odin:21-37), p through this wave's LDS
    // row, o = sum_t p(t) v(t) with DPL dimensions per lane, then the split's
    // (o, m, l).  Score = q.k / sqrt(hd) (forward.odin:158 divides).
    const float div = sqrtf((float)HD);
    const int stride = HD + 2;
    for (int g = wave; g < G; g += WG / WAVE) {
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
    const int nsplit = pos / S::CH + 1;
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

template <int HD>
static hipError_t launch_attn_hd(const AttnArgs &a, int G, hipStream_t st) {
    dim3 grid(a.max_splits, a.n_kv_heads), block(WG);
    switch (G) {
    case 1: hipLaunchKernelGGL((attn_kernel<HD, 1>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((attn_kernel<HD, 2>), grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL((attn_kernel<HD, 4>), grid, block, 0, st, a); break;
    case 8: hipLaunchKernelGGL((attn_kernel<HD, 8>), grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(a.n_heads, HD / WAVE), dim3(WG), 0, st, a);
    return hipGetLastError();
}

int attn_chunk(int head_dim) { return head_dim == 256 ? AttnShape<256>::CH : AttnShape<128>::CH; }
int attn_max_splits() { return ATTN_MAX_SPLITS; }

hipError_t launch_attn(const AttnArgs &a, int head_dim, hipStream_t st) {
    const int G = a.n_heads / a.n_kv_heads;
    if (a.max_splits > ATTN_MAX_SPLITS || a.chunk != attn_chunk(head_dim)) return hipErrorInvalidValue;
    if (head_dim == 128) return launch_attn_hd<128>(a, G, st);
    if (head_dim == 256) return launch_attn_hd<256>(a, G, st);
    return hipErrorInvalidValue;
}

}  // namespace oi
